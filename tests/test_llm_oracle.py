"""Pinning of the oracle's Qwen2 pieces (no GPU): ops.rmsNorm (ora_rms_norm, src/ops.zig:409-427),
ops.siluMul (ora_silu_mul, src/ops.zig:429-439) and Model.forward one token at a time
(Oracle.llm_forward, src/llm.zig:169-216) composed of them with ops.linear over gemm.Q8, the
rotary cache writes (oracle/kv.py) and ops.attentionEx over the transposed cache.

Checks: the f64 closed forms (root mean square; x sigmoid(x) up), both the V-wide and the scalar
tail paths; exact known answers; mutations planted in the f64 forms (the mean of squares taken
as a sum, eps outside the root, the tanh GELU in place of SiLU) that the closed-form checks must
reject; and several decode steps of two sequences against an f64 model of the reference's
forward, with planted mistakes (no rotary positions, rotary over interleaved pairs, the GQA map
taken modulo, q's bias dropped, a self-attention one key short, no output norm), each of which
the bar must reject; and the n-token forward (a prompt batch) against the same model over all
rows at once, with attention past a row's own position (no mask within the batch) rejected.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from oracle import kv as kvo


@pytest.fixture(scope="module")
def ora():
    o = oracle.Oracle(2)
    yield o
    o.close()


def rms64(x, w, eps, sum_not_mean=False, eps_outside=False):
    x = np.asarray(x, np.float64)
    ms = (x * x).sum(axis=-1, keepdims=True)
    if not sum_not_mean:
        ms = ms / x.shape[-1]
    den = np.sqrt(ms) + eps if eps_outside else np.sqrt(ms + eps)
    return x / den * np.asarray(w, np.float64)


def silu64(g, u):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


@pytest.mark.parametrize("m,n,eps", [(5, 896, 1e-6), (3, 100, 1e-6), (2, 1536, 1e-5), (1, 4, 1e-6), (7, 17, 1e-6)])
def test_rms_norm_closed_form(ora, m, n, eps):
    rng = np.random.default_rng(m * 31 + n)
    x = (rng.standard_normal((m, n)) * rng.uniform(0.1, 30, (m, 1))).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    got = ora.rms_norm(x, m, n, w, eps)
    ref = rms64(x, w, eps)
    err = np.max(np.abs(got - ref))
    assert err <= 3e-6 * np.max(np.abs(ref))
    for bad in (rms64(x, w, eps, sum_not_mean=True), rms64(x, w, 1e-1, eps_outside=True)):
        assert np.max(np.abs(got - bad)) > 20 * max(err, 1e-6)


def test_rms_norm_known_answers(ora):
    n = 32
    x = np.tile(np.array([3.0, -3.0], np.float32), (1, n // 2))  # rms 3
    w = np.linspace(-2, 2, n).astype(np.float32)
    got = ora.rms_norm(x, 1, n, w, 0.0)
    assert np.max(np.abs(got[0] - np.sign(x[0]) * w)) <= 2e-7


@pytest.mark.parametrize("size", [16, 33, 160, 4096 + 7])
def test_silu_mul_closed_form_both_paths(ora, size):
    rng = np.random.default_rng(size)
    g = np.linspace(-20, 20, size).astype(np.float32)
    u = rng.standard_normal(size).astype(np.float32)
    got = ora.silu_mul(g, u)
    ref = silu64(g, u)
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) <= 2e-6
    gelu = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3))) * u
    assert np.max(np.abs(got - gelu)) > 1e-3


def test_silu_mul_known_answers(ora):
    g = np.array([0.0] * 16 + [50.0, -50.0, 0.0], np.float32)
    u = np.full(g.size, 3.0, np.float32)
    y = ora.silu_mul(g, u)
    assert np.all(y[:16] == 0.0) and y[18] == 0.0
    assert y[16] == np.float32(150.0) and abs(float(y[17])) < 1e-18


NE, H, HK, NFF, NV, NL, NCTX, BASE, EPS = 64, 4, 2, 96, 80, 2, 16, 1e4, 1e-6


def q8(rng, n, k):
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = (rng.uniform(0.5, 1.5, (n, k // 32)) / 127 / np.sqrt(k) * 2).astype(np.float32)
    return q, s


def model(rng):
    d = NE // H
    layers = []
    for _ in range(NL):
        w = {"wq": q8(rng, NE, NE), "wk": q8(rng, HK * d, NE), "wv": q8(rng, HK * d, NE), "wo": q8(rng, NE, NE),
             "w_gate": q8(rng, NFF, NE), "w_up": q8(rng, NFF, NE), "w_down": q8(rng, NE, NFF),
             "bq": (rng.standard_normal(NE) * 0.3).astype(np.float32),
             "bk": (rng.standard_normal(HK * d) * 0.3).astype(np.float32),
             "bv": (rng.standard_normal(HK * d) * 0.1).astype(np.float32),
             "attn_norm": (1 + 0.1 * rng.standard_normal(NE)).astype(np.float32),
             "ffn_norm": (1 + 0.1 * rng.standard_normal(NE)).astype(np.float32)}
        layers.append(w)
    cos, sin = kvo.rope_tables(NCTX, d, BASE)
    return {"embd": q8(rng, NV, NE), "output": q8(rng, NV, NE),
            "output_norm": (1 + 0.1 * rng.standard_normal(NE)).astype(np.float32), "n_head": H, "n_head_kv": HK,
            "eps": EPS, "cos": cos, "sin": sin, "layers": layers}


def deq(w):
    q, s = w
    return (q.astype(np.float64).reshape(q.shape[0], -1, 32) * s.astype(np.float64)[:, :, None]).reshape(q.shape)


def rope64(x, heads, d, pos, interleaved=False):
    x = x.reshape(heads, d).copy()
    half = d // 2
    for j in range(half):
        ang = pos / BASE ** (2 * j / d)
        c, s = math.cos(ang), math.sin(ang)
        i0, i1 = (2 * j, 2 * j + 1) if interleaved else (j, j + half)
        a, b = x[:, i0].copy(), x[:, i1].copy()
        x[:, i0] = a * c - b * s
        x[:, i1] = a * s + b * c
    return x.reshape(-1)


def forward64(lm, cache, token, pos, bug=None):
    d = NE // H
    x = deq(lm["embd"])[token]
    for li, w in enumerate(lm["layers"]):
        h = rms64(x, w["attn_norm"], EPS)
        q = deq(w["wq"]) @ h + (0.0 if bug == "no_bias" else w["bq"])
        k = deq(w["wk"]) @ h + w["bk"]
        v = deq(w["wv"]) @ h + w["bv"]
        if bug != "no_rope":
            q = rope64(q, H, d, pos, bug == "interleaved")
            k = rope64(k, HK, d, pos, bug == "interleaved")
        cache["k"][li][pos] = k
        cache["v"][li][pos] = v
        end = pos if bug == "short" and pos > 0 else pos + 1
        att = np.zeros(NE)
        for hh in range(H):
            hk = hh % HK if bug == "gqa_mod" else hh // (H // HK)
            kk = cache["k"][li][:end, hk * d:(hk + 1) * d]
            vv = cache["v"][li][:end, hk * d:(hk + 1) * d]
            sc = kk @ q[hh * d:(hh + 1) * d] / math.sqrt(d)
            p = np.exp(sc - sc.max())
            att[hh * d:(hh + 1) * d] = (p / p.sum()) @ vv
        x = x + deq(w["wo"]) @ att
        h = rms64(x, w["ffn_norm"], EPS)
        x = x + deq(w["w_down"]) @ silu64(deq(w["w_gate"]) @ h, deq(w["w_up"]) @ h)
    h = x if bug == "no_output_norm" else rms64(x, lm["output_norm"], EPS)
    return deq(lm["output"]) @ h


def test_llm_forward_against_f64(ora):
    rng = np.random.default_rng(3)
    lm = model(rng)
    d = NE // H
    seqs = []
    for _ in range(2):
        seqs.append(({"kt": np.zeros((NL, HK * d * NCTX), np.float32), "v": np.zeros((NL, NCTX, HK * d), np.float32)},
                     {"k": np.zeros((NL, NCTX, HK * d)), "v": np.zeros((NL, NCTX, HK * d))}))
    worst = 0.0
    for step in range(5):
        for si, (cache, c64) in enumerate(seqs):
            pos = step + 4 * si
            if step == 0 and si == 1:
                for p in range(4):  # sequence 1's earlier tokens
                    t0 = int(rng.integers(0, NV))
                    ora.llm_forward(lm, cache, t0, p)
                    forward64(lm, c64, t0, p)
            tok = int(rng.integers(0, NV))
            before = {"k": c64["k"].copy(), "v": c64["v"].copy()}
            got = ora.llm_forward(lm, cache, tok, pos)
            ref = forward64(lm, c64, tok, pos)
            scale = max(1.0, np.max(np.abs(ref)))
            err = np.max(np.abs(got - ref)) / scale
            worst = max(worst, err)
            assert err <= 2e-5, (step, si, err)
            # the transposed cache column and the value row at pos hold the rotated k and v
            for li in range(NL):
                kt = cache["kt"][li].reshape(HK * d, NCTX)[:, pos]
                assert np.max(np.abs(kt - c64["k"][li][pos])) <= 2e-5 * scale
                assert np.max(np.abs(cache["v"][li][pos] - c64["v"][li][pos])) <= 2e-5 * scale
            if step >= 1:
                for bug in ("no_rope", "interleaved", "gqa_mod", "no_bias", "short", "no_output_norm"):
                    cb = {"k": before["k"].copy(), "v": before["v"].copy()}
                    bad = forward64(lm, cb, tok, pos, bug=bug)
                    assert np.max(np.abs(got - bad)) / scale > 50 * max(err, 1e-7), bug
    print(f"worst relative error {worst:.2e}")
    assert worst < 2e-5


def forward64_batch(lm, cache, toks, pos, bug=None):
    """The reference's forward over n tokens at pos .. pos + n - 1 in f64: each layer over all rows,
    query i attending to keys 0 .. pos + i (bug "noncausal": to all pos + n keys)."""
    d = NE // H
    n = len(toks)
    x = deq(lm["embd"])[list(toks)]
    for li, w in enumerate(lm["layers"]):
        h = rms64(x, w["attn_norm"], EPS)
        q = h @ deq(w["wq"]).T + w["bq"]
        k = h @ deq(w["wk"]).T + w["bk"]
        v = h @ deq(w["wv"]).T + w["bv"]
        for i in range(n):
            q[i] = rope64(q[i], H, d, pos + i)
            k[i] = rope64(k[i], HK, d, pos + i)
        cache["k"][li][pos:pos + n] = k
        cache["v"][li][pos:pos + n] = v
        att = np.zeros((n, NE))
        for i in range(n):
            end = pos + n if bug == "noncausal" else pos + i + 1
            for hh in range(H):
                hk = hh // (H // HK)
                kk = cache["k"][li][:end, hk * d:(hk + 1) * d]
                vv = cache["v"][li][:end, hk * d:(hk + 1) * d]
                sc = kk @ q[i, hh * d:(hh + 1) * d] / math.sqrt(d)
                p = np.exp(sc - sc.max())
                att[i, hh * d:(hh + 1) * d] = (p / p.sum()) @ vv
        x = x + att @ deq(w["wo"]).T
        h = rms64(x, w["ffn_norm"], EPS)
        g = h @ deq(w["w_gate"]).T
        u = h @ deq(w["w_up"]).T
        x = x + (g / (1 + np.exp(-g)) * u) @ deq(w["w_down"]).T
    return deq(lm["output"]) @ rms64(x[-1], lm["output_norm"], EPS)


def test_llm_forward_batch_against_f64(ora):
    """The n-token forward (a prompt batch): the last token's logits and every cache row against
    the f64 model over all rows at once, after a first batch; a batch attending past each row's
    own position (no causal mask within the batch) fails the bar."""
    rng = np.random.default_rng(5)
    lm = model(rng)
    d = NE // H
    cache = {"kt": np.zeros((NL, HK * d * NCTX), np.float32), "v": np.zeros((NL, NCTX, HK * d), np.float32)}
    c64 = {"k": np.zeros((NL, NCTX, HK * d)), "v": np.zeros((NL, NCTX, HK * d))}
    worst = 0.0
    for pos, n in ((0, 5), (5, 7), (12, 1)):
        toks = rng.integers(0, NV, n)
        before = {"k": c64["k"].copy(), "v": c64["v"].copy()}
        got = ora.llm_forward(lm, cache, toks, pos)
        ref = forward64_batch(lm, c64, toks, pos)
        scale = max(1.0, np.max(np.abs(ref)))
        err = np.max(np.abs(got - ref)) / scale
        worst = max(worst, err)
        assert err <= 2e-5, (pos, n, err)
        for li in range(NL):
            kt = cache["kt"][li].reshape(HK * d, NCTX)[:, pos:pos + n].T
            assert np.max(np.abs(kt - c64["k"][li][pos:pos + n])) <= 2e-5 * scale
            assert np.max(np.abs(cache["v"][li][pos:pos + n] - c64["v"][li][pos:pos + n])) <= 2e-5 * scale
        if n > 1:
            bad = forward64_batch(lm, {"k": before["k"].copy(), "v": before["v"].copy()}, toks, pos, bug="noncausal")
            assert np.max(np.abs(got - bad)) / scale > 50 * max(err, 1e-7)
    print(f"worst relative error {worst:.2e}")

