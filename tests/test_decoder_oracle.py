"""Pinning of the oracle's Whisper decoder composition (no GPU): Oracle.decoder_set_audio
(Decoder.setAudio, src/decoder.zig:151-159) and Oracle.decoder_forward (Decoder.forward,
src/decoder.zig:165-205, one token per call), composed of the pinned ops.linear over gemm.Q8,
ops.layerNorm, ops.gelu and ops.attention.

Checks: a token sequence of several steps per window (so the self-attention reads cache rows
written by earlier steps, and windows start at different positions) against an f64 model of the
same steps written from the reference's forward; the cache rows the steps write; and mutations
planted in the f64 model -- a residual dropped, the self-attention ending one key early, the
positional row left out, the cross-attention over the wrong window, the final norm skipped --
each of which the bar must reject.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import pytest

import oracle
from oracle import naive

NS, H, NL, NV, NCTX, NAUD = 64, 2, 2, 96, 12, 40


@pytest.fixture(scope="module")
def ora():
    o = oracle.Oracle(3)
    yield o
    o.close()


def q8(rng, n, k):
    """A gemm.Q8 pair (int8 [n][k], f32 scales [n][k / 32]) of weights ~ N(0, 1/k)."""
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    s = (rng.uniform(0.5, 1.5, (n, k // 32)) / 127 / np.sqrt(k) * 2).astype(np.float32)
    return q, s


def model(rng):
    def vec(n, scale=0.1):
        return (rng.standard_normal(n) * scale).astype(np.float32)

    layers = []
    for _ in range(NL):
        w = {}
        for name in ("q_w", "k_w", "v_w", "o_w", "cq_w", "ck_w", "cv_w", "co_w"):
            w[name] = q8(rng, NS, NS)
        w["mlp0_w"], w["mlp1_w"] = q8(rng, 4 * NS, NS), q8(rng, NS, 4 * NS)
        for name in ("q_b", "v_b", "o_b", "cq_b", "cv_b", "co_b", "mlp1_b"):
            w[name] = vec(NS)
        w["mlp0_b"] = vec(4 * NS)
        for ln in ("attn_ln", "cross_ln", "mlp_ln"):
            w[ln + "_w"], w[ln + "_b"] = 1 + vec(NS), vec(NS)
        layers.append(w)
    return {"te": q8(rng, NV, NS), "pe": rng.standard_normal((NCTX, NS)).astype(np.float32) * 0.5,
            "ln_w": 1 + vec(NS), "ln_b": vec(NS), "n_head": H, "layers": layers}


def deq(w):
    q, s = w
    return (q.astype(np.float64).reshape(q.shape[0], -1, 32) * s.astype(np.float64)[:, :, None]).reshape(q.shape)


def ln64(x, w, b, eps=1e-5):
    mu = x.mean()
    return (x - mu) / np.sqrt(((x - mu) ** 2).mean() + eps) * w.astype(np.float64) + b.astype(np.float64)


def gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def attn64(q, k, v):
    sh = SimpleNamespace(n_q=1, n_kv=k.shape[0], n_head=H, n_head_kv=H, d=NS // H, q_stride=NS, kv_stride=NS,
                         out_stride=NS, kt_stride=0, causal=False)
    return naive.attention_f64(q.reshape(-1), k.reshape(-1), v.reshape(-1), sh)


def forward64(dec, cache, cross, token, pos, bug=None):
    """The reference's forward for one token in f64 (cache: f64 [layer][n_ctx][ns] k and v)."""
    def lin(a, w, b):
        r = deq(w) @ a
        return r if b is None else r + b.astype(np.float64)

    x = deq(dec["te"])[token] + (0.0 if bug == "no_pe" else dec["pe"][pos].astype(np.float64))
    for li, w in enumerate(dec["layers"]):
        xl = ln64(x, w["attn_ln_w"], w["attn_ln_b"])
        q = lin(xl, w["q_w"], w["q_b"])
        cache["k"][li][pos] = lin(xl, w["k_w"], None)
        cache["v"][li][pos] = lin(xl, w["v_w"], w["v_b"])
        end = pos if bug == "short_self" and pos > 0 else pos + 1
        x = x + lin(attn64(q, cache["k"][li][:end], cache["v"][li][:end]), w["o_w"], w["o_b"])
        xl = ln64(x, w["cross_ln_w"], w["cross_ln_b"])
        q = lin(xl, w["cq_w"], w["cq_b"])
        ck, cv = cross[li] if bug != "wrong_window" else cross["other"][li]
        a = lin(attn64(q, ck, cv), w["co_w"], w["co_b"])
        x = a if bug == "no_residual" else x + a
        xl = ln64(x, w["mlp_ln_w"], w["mlp_ln_b"])
        x = x + lin(gelu64(lin(xl, w["mlp0_w"], w["mlp0_b"])), w["mlp1_w"], w["mlp1_b"])
    xl = x if bug == "no_final_ln" else ln64(x, dec["ln_w"], dec["ln_b"])
    return deq(dec["te"]) @ xl


def test_decoder_forward_against_f64(ora):
    rng = np.random.default_rng(11)
    dec = model(rng)
    windows = []
    for w in range(2):
        enc = rng.standard_normal((NAUD, NS)).astype(np.float32)
        cross = ora.decoder_set_audio(enc, NAUD, NS, dec["layers"])
        # setAudio is enc . ck^T and enc . cv^T + cv_b per layer
        for li, (ck, cv) in enumerate(cross):
            lw = dec["layers"][li]
            assert np.max(np.abs(ck - enc.astype(np.float64) @ deq(lw["ck_w"]).T)) <= 1e-5
            assert np.max(np.abs(cv - (enc.astype(np.float64) @ deq(lw["cv_w"]).T + lw["cv_b"]))) <= 1e-5
        cache = {"k": np.zeros((NL, NCTX, NS), np.float32), "v": np.zeros((NL, NCTX, NS), np.float32),
                 "ck": np.stack([c[0] for c in cross]), "cv": np.stack([c[1] for c in cross])}
        c64 = {"k": np.zeros((NL, NCTX, NS)), "v": np.zeros((NL, NCTX, NS))}
        windows.append((cross, cache, c64))
    other = windows[1][0]
    worst = 0.0
    for step in range(4):
        for wi, (cross, cache, c64) in enumerate(windows):
            pos = step + 3 * wi  # window 1 at positions 3..6
            if step == 0 and wi == 1:
                # window 1's rows 0..2 from earlier steps, as a decode that began before this one
                for p in range(3):
                    tok = int(rng.integers(0, NV))
                    ora.decoder_forward(dec, cache, tok, p)
                    forward64(dec, c64, cross, tok, p)
            tok = int(rng.integers(0, NV))
            got = ora.decoder_forward(dec, cache, tok, pos)
            cref = {"k": c64["k"].copy(), "v": c64["v"].copy()}
            ref = forward64(dec, c64, cross, tok, pos)
            scale = max(1.0, np.max(np.abs(ref)))
            err = np.max(np.abs(got - ref)) / scale
            worst = max(worst, err)
            assert err <= 2e-5, (step, wi, err)
            # the step wrote k and v rows at pos, as the f64 model did
            for li in range(NL):
                assert np.max(np.abs(cache["k"][li][pos] - c64["k"][li][pos])) <= 2e-5 * scale
                assert np.max(np.abs(cache["v"][li][pos] - c64["v"][li][pos])) <= 2e-5 * scale
            # planted mistakes are far outside the bar
            if step >= 1:
                bad_cross = dict(enumerate(cross))
                bad_cross["other"] = other if wi == 0 else windows[0][0]
                for bug in ("no_pe", "short_self", "wrong_window", "no_residual", "no_final_ln"):
                    cb = {"k": cref["k"].copy(), "v": cref["v"].copy()}
                    bad = forward64(dec, cb, bad_cross, tok, pos, bug=bug)
                    assert np.max(np.abs(got - bad)) / scale > 50 * max(err, 1e-7), bug
    print(f"worst relative error {worst:.2e}")
    assert worst < 2e-5
