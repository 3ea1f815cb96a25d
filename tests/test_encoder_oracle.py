"""Pinning of the oracle's encoder-layer ops (no GPU): ops.layerNormEps (oracle/attn_oracle.c
ora_layer_norm, src/ops.zig:342-395), ops.gelu (ora_gelu, src/ops.zig:310-340) and one Whisper
encoder layer composed of them with ops.linear and ops.attention (Oracle.encoder_layer,
src/encoder.zig:164-175).

Checks: the f64 closed forms (mean / biased variance normalisation; ggml's tanh GELU); exact
known answers (a constant row normalises to b; gelu(0) = 0, gelu(x) = x once tanh saturates,
gelu(x) - gelu(-x) = x); both GELU paths (16-wide vector and the scalar tail); mutations planted
in the f64 forms (unbiased variance, eps outside the root, the erf GELU, a wrong cubic
coefficient) that the closed-form checks must reject; and the whole layer against an f64
composition of the same steps.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import pytest

import oracle
from oracle import naive


@pytest.fixture(scope="module")
def ora():
    o = oracle.Oracle(3)
    yield o
    o.close()


def ln64(x, w, b, eps=1e-5, ddof=0, eps_outside=False):
    x = x.astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).sum(axis=1, keepdims=True) / (x.shape[1] - ddof)
    den = np.sqrt(var) + eps if eps_outside else np.sqrt(var + eps)
    return (x - mu) / den * w.astype(np.float64) + b.astype(np.float64)


def gelu64(x, cubic=0.044715):
    x = x.astype(np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + cubic * x ** 3)))


def gelu_erf64(x):
    x = x.astype(np.float64)
    return 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))


@pytest.mark.parametrize("m,n,eps", [(7, 384, 1e-5), (3, 512, 1e-5), (65, 768, 1e-12), (2, 100, 1e-5), (1, 4, 1e-5)])
def test_layer_norm_closed_form(ora, m, n, eps):
    rng = np.random.default_rng(m * n)
    x = (rng.standard_normal((m, n)) * rng.uniform(0.1, 20, (m, 1)) + rng.uniform(-5, 5, (m, 1))).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    got = ora.layer_norm(x, m, n, w, b, eps)
    ref = ln64(x, w, b, eps)
    err = np.max(np.abs(got - ref))
    assert err <= 2e-5 * np.max(np.abs(ref))
    # planted mistakes in the f64 form are far outside that bar
    for bad in (ln64(x, w, b, eps, ddof=1), ln64(x, w, b, 1e-1 if eps == 1e-5 else 1e-3, eps_outside=True)):
        assert np.max(np.abs(got - bad)) > 20 * max(err, 1e-6)


def test_layer_norm_known_answers(ora):
    n = 64
    w = np.linspace(-2, 2, n).astype(np.float32)
    b = np.linspace(3, -1, n).astype(np.float32)
    x = np.full((2, n), 7.25, np.float32)
    assert np.array_equal(ora.layer_norm(x, 2, n, w, b), np.stack([b, b]))  # zero deviation -> b exactly
    x = np.tile(np.array([1.0, -1.0], np.float32), (1, n // 2))  # mean 0, var 1
    got = ora.layer_norm(x, 1, n, np.ones(n, np.float32), np.zeros(n, np.float32), 0.0)
    assert np.array_equal(got[0], x[0])


@pytest.mark.parametrize("size", [16, 17, 100, 4096 + 5])
def test_gelu_closed_form_both_paths(ora, size):
    x = np.linspace(-9, 9, size).astype(np.float32)
    got = ora.gelu(x)
    ref = gelu64(x)
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) <= 2e-6
    # the erf GELU and a wrong cubic coefficient differ by far more than that
    assert np.max(np.abs(got - gelu_erf64(x))) > 1e-4
    assert np.max(np.abs(got - gelu64(x, cubic=0.04))) > 1e-4


def test_gelu_known_answers(ora):
    x = np.array([0.0] * 16 + [30.0, 50.0, -30.0, 2.0, -2.0, 0.5, -0.5], np.float32)
    y = ora.gelu(x)
    assert np.all(y[:16] == 0.0)
    assert y[16] == np.float32(30.0) and y[17] == np.float32(50.0) and y[18] == 0.0
    assert abs((float(y[19]) - float(y[20])) - 2.0) <= 1e-6 and abs((float(y[21]) - float(y[22])) - 0.5) <= 1e-6


def layer_weights(rng, ns):
    def f16(n, k):
        return (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16)

    def vec(n, scale=0.1):
        return (rng.standard_normal(n) * scale).astype(np.float32)

    return {"attn_ln_w": 1 + vec(ns), "attn_ln_b": vec(ns), "q_w": f16(ns, ns), "q_b": vec(ns), "k_w": f16(ns, ns),
            "v_w": f16(ns, ns), "v_b": vec(ns), "o_w": f16(ns, ns), "o_b": vec(ns), "mlp_ln_w": 1 + vec(ns),
            "mlp_ln_b": vec(ns), "mlp0_w": f16(4 * ns, ns), "mlp0_b": vec(4 * ns), "mlp1_w": f16(ns, 4 * ns),
            "mlp1_b": vec(ns)}


def layer64(x, n_ctx, ns, n_head, w):
    def lin(a, wn, bn):
        r = a @ w[wn].astype(np.float64).T
        return r if bn is None else r + w[bn].astype(np.float64)

    x = x.astype(np.float64)
    xl = ln64(x, w["attn_ln_w"], w["attn_ln_b"])
    q, k, v = lin(xl, "q_w", "q_b"), lin(xl, "k_w", None), lin(xl, "v_w", "v_b")
    sh = SimpleNamespace(n_q=n_ctx, n_kv=n_ctx, n_head=n_head, n_head_kv=n_head, d=ns // n_head, q_stride=ns,
                         kv_stride=ns, out_stride=ns, kt_stride=0, causal=False)
    att = naive.attention_f64(q.reshape(-1), k.reshape(-1), v.reshape(-1), sh).reshape(n_ctx, ns)
    x = x + lin(att, "o_w", "o_b")
    xl = ln64(x, w["mlp_ln_w"], w["mlp_ln_b"])
    return x + lin(gelu64(lin(xl, "mlp0_w", "mlp0_b")), "mlp1_w", "mlp1_b")


def test_encoder_layer_against_f64(ora):
    rng = np.random.default_rng(1)
    n_ctx, ns, n_head = 70, 64, 2
    w = layer_weights(rng, ns)
    x = rng.standard_normal((n_ctx, ns)).astype(np.float32)
    got = ora.encoder_layer(x, n_ctx, ns, n_head, w)
    ref = layer64(x, n_ctx, ns, n_head, w)
    assert np.max(np.abs(got - ref)) <= 1e-4 * max(1.0, np.max(np.abs(ref)))
