"""Pinning of the oracle's ops.linear with f16 weights (oracle/attn_oracle.c, ora_linear_f16:
src/ops.zig:283-306, src/gemm.zig:27-137).

Checks: the reference's own tests at their shapes and tolerance (src/gemm.zig:412-429 "nt block
with f16 weights", src/ops.zig:611-636 "linear agrees with a plain loop", here with f16
weights); the f64 closed form on shapes that take every path (the serial small-op path, 4x4
tiles, the 1x4 row tail, the single-column tail, the scalar K tail, several pool tasks);
exact known answers (identity weights, one-hot weights, zero weights with a bias); and the f16
widening on every one of the 65536 bit patterns.
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


def ref64(x, w, b, m, k, n):
    out = x.reshape(m, k).astype(np.float64) @ w.reshape(n, k).astype(np.float64).T
    if b is not None:
        out += b.astype(np.float64)[None, :]
    return out


def uni(seed, n):
    return (np.random.default_rng(seed).random(n) - 0.5).astype(np.float32)


def test_reference_nt_block_f16_test(ora):
    """src/gemm.zig:412-429: m=5, n=6, k=2V+3, values in [-0.5, 0.5), 1e-4 abs."""
    m, n, k = 5, 6, 2 * 16 + 3
    x, w = uni(1, m * k), uni(2, n * k).astype(np.float16)
    out = ora.linear_f16(x, m, k, w, None, n)
    assert np.max(np.abs(out - ref64(x, w, None, m, k, n).reshape(-1))) <= 1e-4


def test_reference_linear_test(ora):
    """src/ops.zig:611-636 at its shape (m=70, k=37, n=133, bias, 3 threads), f16 weights, 1e-4 abs."""
    m, k, n = 70, 37, 133
    x, w, b = uni(3, m * k), uni(4, n * k).astype(np.float16), uni(5, n)
    out = ora.linear_f16(x, m, k, w, b, n)
    assert np.max(np.abs(out - ref64(x, w, b, m, k, n).reshape(-1))) <= 1e-4


@pytest.mark.parametrize("m,k,n", [(1, 8, 1), (3, 24, 5), (4, 16, 4), (7, 40, 9), (64, 384, 128), (130, 512, 389),
                                   (1500, 384, 64)])
def test_closed_form(ora, m, k, n):
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = (rng.standard_normal(n * k) / np.sqrt(k)).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float32)
    out = ora.linear_f16(x, m, k, w, b, n)
    ref = ref64(x, w, b, m, k, n).reshape(-1)
    assert np.max(np.abs(out - ref)) <= 2e-5 * np.sqrt(k)


def test_known_answers(ora):
    m, k = 9, 48
    x = np.random.default_rng(6).standard_normal(m * k).astype(np.float32)
    eye = np.eye(k, dtype=np.float16)
    assert np.array_equal(ora.linear_f16(x, m, k, eye, None, k), x)  # identity weights copy x exactly
    onehot = np.zeros((3, k), np.float16)
    onehot[0, 5] = 1
    onehot[1, 47] = 2
    onehot[2, 0] = -0.5
    out = ora.linear_f16(x, m, k, onehot, None, 3).reshape(m, 3)
    xm = x.reshape(m, k)
    assert np.array_equal(out[:, 0], xm[:, 5]) and np.array_equal(out[:, 1], 2 * xm[:, 47])
    assert np.array_equal(out[:, 2], -0.5 * xm[:, 0])
    b = np.arange(7, dtype=np.float32)
    assert np.array_equal(ora.linear_f16(x, m, k, np.zeros((7, k), np.float16), b, 7).reshape(m, 7), np.tile(b, (m, 1)))


def test_f16_widening_every_bit_pattern(ora):
    """Weights of every f16 bit pattern (finite ones), one per output column, against x = 1."""
    bits = np.arange(0x10000, dtype=np.uint16)
    vals = bits.view(np.float16)
    finite = np.isfinite(vals)
    w = vals[finite].reshape(-1, 1)
    w8 = np.zeros((w.shape[0], 8), np.float16)
    w8[:, 0] = w[:, 0]
    x = np.zeros(8, np.float32)
    x[0] = 1.0
    out = ora.linear_f16(x, 1, 8, w8, None, w8.shape[0])
    assert np.array_equal(out, w8[:, 0].astype(np.float32))
