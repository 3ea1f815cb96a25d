"""The seeded input generator and the algorithmic work of the five benchmark workloads."""
from __future__ import annotations

import numpy as np

from zwhisper_amd import workloads as W


def test_splitmix64_known_answer():
    # SplitMix64 reference vector: seed 0 -> e220a8397b1dcdaf, 6e789e6aa1b965f4, 06c45d188009454f
    assert [int(x) for x in W.splitmix64(0, 3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_uniform_and_normal_are_deterministic_and_well_shaped():
    u = W.uniform(7, 200_000)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.005
    z = W.normal(7, 400_001)
    assert z.dtype == np.float32 and z.size == 400_001
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1.0) < 0.01
    assert np.array_equal(W.normal(7, 10), W.normal(7, 10)[:10])
    assert not np.array_equal(W.normal(7, 10), W.normal(8, 10))


def test_rope_is_a_rotation():
    x = W.normal(5, 6 * 3 * 64).reshape(6, 3, 64)
    pos = np.arange(6)
    y = W.apply_rope(x, pos, 64)
    # position 0 is the identity; every (k, k + d/2) pair keeps its length
    assert np.array_equal(y[0], x[0])
    nx = x[..., :32] ** 2 + x[..., 32:] ** 2
    ny = y[..., :32] ** 2 + y[..., 32:] ** 2
    assert np.allclose(nx, ny, rtol=1e-5, atol=1e-5)
    # position 1, pair 0 turns by exactly 1 radian (inverse frequency theta^0 = 1)
    a, b = x[1, 0, 0], x[1, 0, 32]
    assert np.isclose(y[1, 0, 0], a * np.cos(1.0) - b * np.sin(1.0), atol=1e-6)
    assert np.isclose(y[1, 0, 32], a * np.sin(1.0) + b * np.cos(1.0), atol=1e-6)


def test_cache_lengths_in_range():
    l3, l5 = W.kv_lengths(3), W.kv_lengths(5)
    assert l3.shape == (32,) and l3.min() >= 1 and l3.max() <= 448
    assert l5.shape == (64,) and l5.min() >= 1024 and l5.max() <= 4096


def test_algorithmic_work_matches_the_published_formulas():
    assert W.algorithmic_work(1) == 4 * 1500 * 1500 * 64 * 6 == 3.456e9
    assert W.algorithmic_work(2) == 16 * 4 * 1500 * 1500 * 64 * 8
    assert W.algorithmic_work(4) == 4 * 64 * 14 * (2048 * 2049 // 2)
    l3 = W.kv_lengths(3)
    c3 = float(np.sum(2 * l3 * 768 * 4) + 32 * 2 * 1500 * 768 * 4 + 32 * 4 * 768 * 4)
    assert W.algorithmic_work(3) == c3 and 330e6 < c3 < 350e6
    l5 = W.kv_lengths(5)
    c5 = float(np.sum(2 * 2 * 128 * 4 * l5) + 64 * 2 * 1536 * 4)
    assert W.algorithmic_work(5) == c5 and 300e6 < c5 < 380e6


def test_transposed_layout():
    kl = W.normal(9, 5 * 2 * 4).reshape(5, 2, 4)
    kt = W.to_kt(kl, 8)
    assert kt.shape == (2, 4, 8)
    assert np.array_equal(kt[1, 3, :5], kl[:, 1, 3]) and np.all(kt[:, :, 5:] == 0)
