"""Pins the CPU oracle (oracle/attn_oracle.c) and the f64 closed form (oracle/naive.py).

What pins what:
* the reference's own tests: expVec vs exp (src/ops.zig:706-716), pvBlock vs a naive loop
  (src/gemm.zig:431-448), attention vs a naive loop at n_q=70, n_kv=90, 2 heads, d=32, causal
  and not (src/ops.zig:655-704);
* closed forms that fix the scale 1/sqrt(d), the causal rule j <= n_kv - n_q + i, the GQA map
  h -> h / (n_head / n_head_kv) and the layouts, so a wrong constant, index or transposed operand
  fails at least one of them (the mutation tests at the end plant such mistakes);
* an independent pure-Python loop on tiny shapes;
* invariants (key permutation, head independence, row-major vs transposed K, convex hull);
* the committed golden fixtures (tests/golden/).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from _golden import head_columns_mask, load_cases
from oracle import naive
from zwhisper_amd import workloads as W
from zwhisper_amd.ops import AttnShape


@pytest.fixture(scope="module")
def ora():
    o = oracle.Oracle(2)
    yield o
    o.close()


def shape(n_q, n_kv, h, hkv, d, causal, kt=None, qs=None, kvs=None, os_=None):
    return AttnShape(n_q, n_kv, h, hkv, d, qs or h * d, kvs or hkv * d, os_ or h * d, causal, kt)


def rand_inputs(sh: AttnShape, seed: int):
    q = W.normal(seed, max(sh.q_len(), 1))
    kvd = sh.n_head_kv * sh.d
    kl = W.normal(seed + 1, sh.n_kv * kvd).reshape(sh.n_kv, sh.n_head_kv, sh.d)
    if sh.kt_stride:
        k = W.to_kt(kl, sh.kt_stride).reshape(-1)
    else:
        k = np.zeros(max(sh.k_len(), 1), np.float32)
        for t in range(sh.n_kv):
            k[t * sh.kv_stride: t * sh.kv_stride + kvd] = kl[t].reshape(-1)
    v = W.normal(seed + 2, max(sh.v_len(), 1))
    return q, k, v


# ---------------------------------------------------------------------------------------------
# the reference's own tests


def test_exp_vec_matches_exp_reference_range():
    """src/ops.zig:706-716: V points over [-10, 10), relative error <= 1e-6."""
    x = (-10.0 + 20.0 * np.arange(16) / 16).astype(np.float32)
    got = oracle.exp_vec(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    assert np.max(np.abs(got - want) / want) <= 1e-6


def test_exp_vec_wide_range_and_special_values():
    x = np.linspace(-87.0, 88.0, 16 * 200, dtype=np.float32)
    got = oracle.exp_vec(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    assert np.max(np.abs(got - want) / want) <= 2e-6
    special = oracle.exp_vec(np.array([0.0] + [-200.0] + [1.0] * 14, dtype=np.float32))
    assert special[0] == 1.0  # r = 0: the polynomial gives exactly 1
    assert special[1] < 2e-38  # clamped at -87.3
    assert abs(special[2] - math.e) <= 1e-6 * math.e


@pytest.mark.parametrize("m,t,d", [(6, 11, 32), (7, 33, 64), (9, 5, 128), (1, 1, 16), (4, 0, 32)])
def test_pv_block_matches_naive(m, t, d):
    """src/gemm.zig:431-448 (m=6, t=11, d=2V) plus the tail-row, w<4 and d=128 paths."""
    p = W.uniform(50 + m, m * t).reshape(m, t).astype(np.float32)
    v = W.uniform_centered(60 + t, t * d).reshape(t, d)
    got = oracle.pv_block(p, v)
    want = p.astype(np.float64) @ v.astype(np.float64)
    assert np.max(np.abs(got - want), initial=0.0) <= 1e-4


@pytest.mark.parametrize("n", [1, 15, 16, 37, 1500])
def test_softmax_row(n):
    x = (W.normal(70 + n, n) * 3).astype(np.float32)
    got = oracle.softmax_row(x).astype(np.float64)
    e = np.exp(x.astype(np.float64) - x.max())
    want = e / e.sum()
    assert np.max(np.abs(got - want)) <= 1e-6
    assert abs(got.sum() - 1.0) <= 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_reference_attention_test_shape(ora, causal):
    """src/ops.zig:655-704: n_q=70, n_kv=90, 2 heads, d=2V, inputs U[-0.5, 0.5), 1e-4 abs."""
    n_q, n_kv, h = 70, 90, 2
    ns = 2 * 16 * h
    q = W.uniform_centered(9, n_q * ns)
    k = W.uniform_centered(10, n_kv * ns)
    v = W.uniform_centered(11, n_kv * ns)
    got = ora.attention(q, k, v, n_q, n_kv, ns, h, causal)
    sh = shape(n_q, n_kv, h, h, ns // h, causal)
    want = naive.attention_f64(q, k, v, sh)
    assert np.max(np.abs(got - want)) <= 1e-4
    assert np.max(np.abs(got - want)) <= 2e-6  # what the restatement actually achieves


def _python_loop_attention(q, k, v, n_q, n_kv, h, d, causal):
    """Independent brute force in plain Python floats (row-major everything, MHA)."""
    ns = h * d
    out = [0.0] * (n_q * ns)
    scale = 1.0 / math.sqrt(d)
    for hh in range(h):
        for i in range(n_q):
            limit = n_kv - n_q + i + 1 if causal else n_kv
            s = [sum(float(q[i * ns + hh * d + p]) * float(k[t * ns + hh * d + p]) for p in range(d)) * scale
                 for t in range(limit)]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            tot = sum(e)
            for p in range(d):
                out[i * ns + hh * d + p] = sum(e[t] / tot * float(v[t * ns + hh * d + p]) for t in range(limit))
    return np.array(out)


@pytest.mark.parametrize("causal", [False, True])
def test_naive_and_oracle_match_python_loops(ora, causal):
    n_q, n_kv, h, d = 5, 9, 2, 16
    q = W.normal(1, n_q * h * d)
    k = W.normal(2, n_kv * h * d)
    v = W.normal(3, n_kv * h * d)
    want = _python_loop_attention(q, k, v, n_q, n_kv, h, d, causal)
    sh = shape(n_q, n_kv, h, h, d, causal)
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - want)) <= 1e-12
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - want)) <= 2e-6


# ---------------------------------------------------------------------------------------------
# closed forms


def test_single_key_returns_value_row(ora):
    for causal, n_q in ((True, 1), (False, 3)):
        sh = shape(n_q, 1, 3, 3, 32, causal)
        q, k, v = rand_inputs(sh, 100)
        want = np.tile(v[: 3 * 32], n_q)
        assert np.array_equal(naive.attention_f64(q, k, v, sh), want.astype(np.float64))
        assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - want)) <= 1e-6


@pytest.mark.parametrize("n_q,n_kv", [(4, 4), (3, 10), (1, 7)])
def test_zero_query_averages_visible_values(ora, n_q, n_kv):
    """q = 0 makes every visible score equal: query i averages keys 0 .. n_kv - n_q + i."""
    h, d = 2, 16
    sh = shape(n_q, n_kv, h, h, d, True)
    q = np.zeros(sh.q_len(), np.float32)
    _, k, v = rand_inputs(sh, 200)
    vv = v.reshape(n_kv, h * d).astype(np.float64)
    want = np.stack([vv[: n_kv - n_q + i + 1].mean(axis=0) for i in range(n_q)]).reshape(-1)
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - want)) <= 1e-12
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - want)) <= 1e-6
    sh_nc = shape(n_q, n_kv, h, h, d, False)
    want_nc = np.tile(vv.mean(axis=0), n_q)
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh_nc) - want_nc)) <= 1e-6


@pytest.mark.parametrize("d", [32, 64, 128])
def test_two_key_closed_form_pins_the_scale(ora, d):
    """q = e0, k0 = 8 e0, k1 = 0: scores 8/sqrt(d) and 0, out = (e^s v0 + v1) / (e^s + 1)."""
    sh = shape(1, 2, 1, 1, d, False)
    q = np.zeros(d, np.float32)
    q[0] = 1.0
    k = np.zeros(2 * d, np.float32)
    k[0] = 8.0
    v = W.normal(300 + d, 2 * d)
    s = 8.0 / math.sqrt(d)
    want = (math.exp(s) * v[:d].astype(np.float64) + v[d:].astype(np.float64)) / (math.exp(s) + 1.0)
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - want)) <= 1e-7
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - want)) <= 1e-6


def test_dominant_key_selects_its_value(ora):
    n_kv, d = 50, 64
    sh = shape(1, n_kv, 1, 1, d, False)
    q = np.zeros(d, np.float32)
    q[3] = 1.0
    k = (W.normal(400, n_kv * d) * 0.1).astype(np.float32)
    k[17 * d + 3] = 400.0  # score 50 above the rest
    v = W.normal(401, n_kv * d)
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - v[17 * d: 18 * d])) <= 1e-6


def test_gqa_head_map(ora):
    """Value rows of KV head j are all j + 1, so output head h must be h // (H / H_kv) + 1."""
    h, hkv, d, n_kv = 6, 3, 32, 20
    sh = shape(4, n_kv, h, hkv, d, True)
    q, k, _ = rand_inputs(sh, 500)
    v = np.tile(np.repeat(np.arange(1, hkv + 1, dtype=np.float32), d), n_kv)
    want = np.tile(np.repeat(np.arange(h) // (h // hkv) + 1.0, d), 4)
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - want)) <= 1e-12
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - want)) <= 1e-6


# ---------------------------------------------------------------------------------------------
# invariants


def test_transposed_and_row_major_keys_agree(ora):
    sh_rm = shape(37, 300, 14, 2, 64, True)
    sh_kt = shape(37, 300, 14, 2, 64, True, kt=304)
    q = W.normal(1, sh_rm.q_len())
    kl = W.normal(2, 300 * 2 * 64).reshape(300, 2, 64)
    v = W.normal(3, sh_rm.v_len())
    a = ora.attention_ex(q, kl.reshape(-1), v, sh_rm)
    b = ora.attention_ex(q, W.to_kt(kl, 304).reshape(-1), v, sh_kt)
    assert np.array_equal(a, b)
    assert np.max(np.abs(naive.attention_f64(q, kl.reshape(-1), v, sh_rm)
                         - naive.attention_f64(q, W.to_kt(kl, 304).reshape(-1), v, sh_kt))) == 0.0


def test_key_permutation_invariance(ora):
    sh = shape(10, 40, 2, 2, 32, False)
    q, k, v = rand_inputs(sh, 600)
    perm = np.random.default_rng(0).permutation(40)
    k2 = k.reshape(40, -1)[perm].reshape(-1)
    v2 = v.reshape(40, -1)[perm].reshape(-1)
    assert np.max(np.abs(ora.attention_ex(q, k, v, sh) - ora.attention_ex(q, k2, v2, sh))) <= 1e-6


def test_heads_are_independent(ora):
    sh = shape(8, 30, 3, 3, 32, True)
    q, k, v = rand_inputs(sh, 700)
    a = ora.attention_ex(q, k, v, sh).reshape(8, 3, 32)
    q2 = q.copy().reshape(8, 3, 32)
    q2[:, 1, :] *= -3.0
    b = ora.attention_ex(q2.reshape(-1), k, v, sh).reshape(8, 3, 32)
    assert np.array_equal(a[:, 0], b[:, 0]) and np.array_equal(a[:, 2], b[:, 2])
    assert not np.allclose(a[:, 1], b[:, 1])


def test_output_gaps_untouched_and_convex_hull(ora):
    sh = shape(9, 33, 2, 2, 32, True, qs=96, kvs=80, os_=72)
    q, k, v = rand_inputs(sh, 800)
    out = np.full(sh.out_len(), 7.25, np.float32)
    ora.attention_ex(q, k, v, sh, out=out)
    m = head_columns_mask(sh)
    assert np.all(out[~m] == 7.25)
    got = out[m].reshape(9, 2, 32)
    vv = np.stack([v[t * 80: t * 80 + 64] for t in range(33)]).reshape(33, 2, 32)
    for i in range(9):
        vis = vv[: 33 - 9 + i + 1]
        assert np.all(got[i] <= vis.max(axis=0) + 1e-6) and np.all(got[i] >= vis.min(axis=0) - 1e-6)


def test_oracle_rejects_what_the_reference_asserts(ora):
    with pytest.raises(ValueError):
        ora.attention_ex(*rand_inputs(shape(2, 3, 2, 2, 24, False), 1), shape(2, 3, 2, 2, 24, False))  # d % V
    with pytest.raises(ValueError):
        ora.attention_ex(*rand_inputs(shape(2, 3, 3, 2, 32, False), 1), shape(2, 3, 3, 2, 32, False))  # H % Hkv
    with pytest.raises(ValueError):
        ora.attention_ex(*rand_inputs(shape(4, 3, 2, 2, 32, True), 1), shape(4, 3, 2, 2, 32, True))  # n_kv < n_q


def test_oracle_multithreaded_equals_single_thread():
    sh = shape(200, 300, 4, 2, 64, True, kt=304)
    q, k, v = rand_inputs(sh, 900)
    with oracle.Oracle(1) as o1, oracle.Oracle(4) as o4:
        assert np.array_equal(o1.attention_ex(q, k, v, sh), o4.attention_ex(q, k, v, sh))


# ---------------------------------------------------------------------------------------------
# golden fixtures

CASES = load_cases()


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_oracle_matches_golden(ora, case):
    got = ora.attention_ex(case.q, case.k, case.v, case.shape)
    m = head_columns_mask(case.shape)
    assert np.max(np.abs(got[m] - case.expected[m]), initial=0.0) <= 1e-5


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_golden_expected_is_the_f64_closed_form(case):
    assert np.max(np.abs(naive.attention_f64(case.q, case.k, case.v, case.shape) - case.expected), initial=0.0) <= 1e-12


# ---------------------------------------------------------------------------------------------
# mutation checks: a planted mistake in the f64 form must fail the closed forms above


def test_planted_wrong_scale_is_caught(monkeypatch):
    monkeypatch.setattr(naive, "_f32_scale", lambda d: 1.0 / d)
    sh = shape(1, 2, 1, 1, 64, False)
    q = np.zeros(64, np.float32)
    q[0] = 1.0
    k = np.zeros(128, np.float32)
    k[0] = 8.0
    v = W.normal(364, 128)
    s = 8.0 / 8.0
    want = (math.exp(s) * v[:64].astype(np.float64) + v[64:].astype(np.float64)) / (math.exp(s) + 1.0)
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - want)) > 1e-3


def test_planted_off_by_one_mask_is_caught():
    sh = shape(3, 10, 2, 2, 16, True)
    q = np.zeros(sh.q_len(), np.float32)
    _, k, v = rand_inputs(sh, 200)
    vv = v.reshape(10, 32).astype(np.float64)
    wrong = np.stack([vv[: 10 - 3 + i].mean(axis=0) for i in range(3)]).reshape(-1)  # j < limit - 1
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - wrong)) > 1e-3


def test_planted_wrong_gqa_map_is_caught():
    h, hkv, d = 6, 3, 32
    sh = shape(2, 5, h, hkv, d, False)
    q, k, _ = rand_inputs(sh, 500)
    v = np.tile(np.repeat(np.arange(1, hkv + 1, dtype=np.float32), d), 5)
    wrong = np.tile(np.repeat(np.arange(h) % hkv + 1.0, d), 2)  # h % H_kv instead of h / group
    assert np.max(np.abs(naive.attention_f64(q, k, v, sh) - wrong)) >= 1.0
