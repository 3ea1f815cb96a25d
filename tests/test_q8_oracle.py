"""Pinning of the oracle's int8 block weights: Q8.quantize (oracle/attn_oracle.c ora_q8_quantize,
src/gemm.zig:209-230) and ops.linear over them (ora_linear_q8: src/ops.zig:283-306, ntBlockQ /
micro4x4Q / dotQ src/gemm.zig:274-351).

Checks: the reference's own test at its shape and tolerances (src/gemm.zig:366-391, "int8 block
matches f32 within quantization error": m=6, n=7, k=64, values in [-0.5, 0.5), 0.02 on the
product, 0.005 on a dequantized row); the f64 closed form over the dequantized weights on shapes
that take every path (serial small-op path, 4x4 tiles, row tail, column tail, pool tasks, bias);
exact known answers (one-hot weights, zero scales); and the quantizer's defining properties
(|q| <= 127, the block's absmax maps to +-127, |w - q s| <= s/2, all-zero blocks, rounding half
away from zero).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


@pytest.fixture(scope="module")
def ora():
    o = oracle.Oracle(3)
    yield o
    o.close()


def uni(seed, shape):
    return (np.random.default_rng(seed).random(shape) - 0.5).astype(np.float32)


def test_reference_int8_block_test(ora):
    m, n, k = 6, 7, 64
    a = uni(11, (m, k))
    w = uni(12, (n, k)).astype(np.float16)
    q, s = oracle.q8_quantize(w, n, k)
    c = ora.linear_q8(a, m, k, q, s, None, n).reshape(m, n)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(c - ref)) <= 0.02
    row2 = oracle.q8_dequantize(q, s)[2]
    assert np.max(np.abs(row2 - w[2].astype(np.float32))) <= 0.005


@pytest.mark.parametrize("m,k,n", [(1, 32, 1), (3, 64, 5), (4, 32, 4), (7, 96, 9), (64, 384, 128), (130, 512, 389),
                                   (1, 768, 2000), (32, 768, 515)])
def test_closed_form(ora, m, k, n):
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    q, s = oracle.q8_quantize(w, n, k)
    out = ora.linear_q8(x, m, k, q, s, b, n).reshape(m, n)
    ref = x.astype(np.float64) @ oracle.q8_dequantize(q, s).astype(np.float64).T + b
    assert np.max(np.abs(out - ref)) <= 2e-5 * np.sqrt(k)


def test_known_answers(ora):
    m, k = 9, 64
    x = np.random.default_rng(6).standard_normal((m, k)).astype(np.float32)
    q = np.zeros((3, k), np.int8)
    s = np.zeros((3, k // 32), np.float32)
    q[0, 5], s[0, 0] = 1, 0.75        # one weight of 0.75 in block 0
    q[1, 40], s[1, 1] = -127, 0.001   # -0.127 in block 1
    q[2, 63], s[2, 1] = 1, 1.0
    out = ora.linear_q8(x, m, k, q, s, None, 3).reshape(m, 3)
    assert np.array_equal(out[:, 0], x[:, 5] * np.float32(0.75))
    assert np.array_equal(out[:, 1], (x[:, 40] * np.float32(-127)) * np.float32(0.001))
    assert np.array_equal(out[:, 2], x[:, 63])
    b = np.arange(4, dtype=np.float32)
    z = ora.linear_q8(x, m, k, np.ones((4, k), np.int8), np.zeros((4, 2), np.float32), b, 4).reshape(m, 4)
    assert np.array_equal(z, np.tile(b, (m, 1)))


def test_quantize_properties():
    rng = np.random.default_rng(3)
    n, k = 50, 256
    w = (rng.standard_normal((n, k)) * rng.random((n, 1)) * 3).astype(np.float32)
    w[7, 32:64] = 0  # an all-zero block
    q, s = oracle.q8_quantize(w, n, k)
    assert q.dtype == np.int8 and s.shape == (n, k // 32)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    blocks = w.reshape(n, k // 32, 32)
    amax = np.abs(blocks).max(axis=2)
    np.testing.assert_array_equal(s, (amax / np.float32(127)).astype(np.float32))
    qb = q.reshape(n, k // 32, 32).astype(np.int32)
    at = np.abs(blocks).argmax(axis=2)
    top = np.take_along_axis(qb, at[..., None], axis=2)[..., 0]
    nz = amax > 0
    assert np.all(np.abs(top[nz]) == 127)
    err = np.abs(blocks - qb * s[..., None])
    assert np.all(err <= s[..., None] * (0.5 + 1e-5))
    assert s[7, 1] == 0 and np.all(q[7, 32:64] == 0)


def test_quantize_rounds_half_away_from_zero():
    w = np.zeros((1, 32), np.float32)
    w[0, :8] = [127.0, 0.5, -0.5, 2.5, -2.5, 1.5, -1.49, 126.5]
    q, s = oracle.q8_quantize(w, 1, 32)
    assert s[0, 0] == 1.0
    assert q[0, :8].tolist() == [127, 1, -1, 3, -3, 2, -1, 127]


def test_f16_input_widens_exactly():
    """Quantizing an f16 matrix equals quantizing its exact f32 widening (src/gemm.zig:215)."""
    w = uni(9, (5, 64)).astype(np.float16)
    q1, s1 = oracle.q8_quantize(w, 5, 64)
    q2, s2 = oracle.q8_quantize(w.astype(np.float32), 5, 64)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
