"""Host side of the int8 block weights (no GPU): zwhisper_amd.Q8, the mirror of gemm.Q8
(src/gemm.zig:196-266).  Q8.quantize must give the oracle's int8 and scales bit for bit (the
oracle's quantizer is pinned in tests/test_q8_oracle.py), Q8.from_q8_0 must read GGUF q8_0 blocks
as src/gemm.zig:232-248 does, and Q8.row must dequantize as src/gemm.zig:255-263.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import zwhisper_amd as z


@pytest.mark.parametrize("n,k,dtype", [(7, 64, np.float16), (33, 96, np.float32), (128, 1536, np.float16)])
def test_quantize_matches_oracle(n, k, dtype):
    rng = np.random.default_rng(n * k)
    w = (rng.standard_normal((n, k)) * rng.uniform(1e-3, 10, (n, 1))).astype(dtype)
    w[0, :32] = 0                 # an all-zero block: scale 0, q 0
    w[1, :32] = np.arange(32) - 16  # exact halves after scaling: ties round away from zero
    got = z.Q8.quantize(w, n, k)
    q, s = oracle.q8_quantize(w, n, k)
    assert np.array_equal(got.q, q)
    assert np.array_equal(got.scales.view(np.uint32), s.view(np.uint32))


def test_ties_away_from_zero():
    """127 * v / amax landing on x.5 rounds away from zero, as Zig's @round."""
    w = np.zeros((1, 32), np.float32)
    w[0, 0] = 127.0
    w[0, 1] = 2.5
    w[0, 2] = -2.5
    w[0, 3] = 0.5
    got = z.Q8.quantize(w, 1, 32)
    assert list(got.q[0, :4]) == [127, 3, -3, 1]
    assert got.scales[0, 0] == np.float32(1.0)


def test_from_q8_0_and_row():
    n, k = 3, 64
    rng = np.random.default_rng(2)
    q = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sc16 = rng.uniform(0.001, 0.1, (n, k // 32)).astype(np.float16)
    blob = bytearray()
    for i in range(n):
        for b in range(k // 32):
            blob += sc16[i, b].tobytes() + q[i, 32 * b:32 * b + 32].tobytes()
    w = z.Q8.from_q8_0(bytes(blob), n, k)
    assert np.array_equal(w.q, q)
    assert np.array_equal(w.scales, sc16.astype(np.float32))
    for i in range(n):
        assert np.array_equal(w.row(i), oracle.q8_dequantize(q, sc16.astype(np.float32))[i])


def test_k_must_be_a_block_multiple():
    with pytest.raises(z.ZwgError, match="multiple of 32"):
        z.Q8.quantize(np.zeros((2, 48), np.float32), 2, 48)
