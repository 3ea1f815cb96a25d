"""Pinning of oracle/kv.py, the CPU restatement of the reference's cache writes
(src/llm.zig:128-137, :182-190, :221-238; src/decoder.zig:182-183).

Every check compares against something the restatement does not compute itself: textbook
values (cos/sin of integers, the Pythagorean identity), invariants of a rotation (norms, the
identity at position 0, composition, relative positions), the exact NeoX pairing on one-hot
inputs, and an independent transpose.  A planted mistake (GPT-J interleaved pairs instead of
NeoX halves) is shown to fail the pairing check.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import kv as okv

BASE = 1.0e6  # qwen2.rope.freq_base default, src/llm.zig:101


def rng_f32(seed: int, *shape: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("d", [64, 128])
def test_tables_textbook_values(d):
    cos, sin = okv.rope_tables(512, d, BASE)
    # position 0: no rotation at all
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # column 0 has frequency 1, so its angle is the position itself
    for p in (1, 2, 3, 100, 511):
        assert cos[p, 0] == np.float32(math.cos(p)) and sin[p, 0] == np.float32(math.sin(p))
    # cos^2 + sin^2 = 1 to f32 rounding everywhere
    assert np.max(np.abs(cos.astype(np.float64) ** 2 + sin.astype(np.float64) ** 2 - 1.0)) < 4e-7


@pytest.mark.parametrize("d", [64, 128])
def test_tables_frequencies(d):
    """At position 1 the angle of column i is base^(-2i/d): a wrong exponent (i/d, or d/2 in the
    denominator) or a wrong base moves it by orders of magnitude."""
    cos, sin = okv.rope_tables(2, d, BASE)
    for i in range(d // 2):
        ang = math.atan2(float(sin[1, i]), float(cos[1, i]))
        want = BASE ** (-2.0 * i / d)
        assert abs(ang - want) <= 2e-7 + 1e-6 * want, (i, ang, want)


def test_rope_identity_at_position_zero():
    cos, sin = okv.rope_tables(4, 128, BASE)
    x = rng_f32(1, 3, 12 * 128)
    y = x.copy()
    okv.rope(y, 3, 12, 128, [0, 0, 0], cos, sin)
    assert np.array_equal(x, y)


def test_rope_neox_pairing_on_one_hot():
    """e_j rotates into dims j and j + d/2 only (NeoX halves, src/llm.zig:232-235)."""
    d, half, p = 64, 32, 37
    cos, sin = okv.rope_tables(64, d, BASE)
    for j in (0, 5, half - 1):
        x = np.zeros(d, np.float32)
        x[j] = 1.0
        okv.rope(x, 1, 1, d, [p], cos, sin)
        want = np.zeros(d, np.float32)
        want[j] = cos[p, j]
        want[j + half] = sin[p, j]
        assert np.array_equal(x, want)
        x = np.zeros(d, np.float32)
        x[j + half] = 1.0
        okv.rope(x, 1, 1, d, [p], cos, sin)
        want = np.zeros(d, np.float32)
        want[j] = -sin[p, j]
        want[j + half] = cos[p, j]
        assert np.array_equal(x, want)


def _rope_interleaved(x, d, p, cos, sin):
    """A planted mistake: GPT-J style pairs (2j, 2j+1) instead of (j, j + d/2)."""
    for j in range(d // 2):
        a, b = x[2 * j], x[2 * j + 1]
        x[2 * j] = a * cos[p, j] - b * sin[p, j]
        x[2 * j + 1] = a * sin[p, j] + b * cos[p, j]


def test_pairing_check_catches_interleaved_pairs():
    d, p = 64, 37
    cos, sin = okv.rope_tables(64, d, BASE)
    x = np.zeros(d, np.float32)
    x[0] = 1.0
    _rope_interleaved(x, d, p, cos, sin)
    want = np.zeros(d, np.float32)
    want[0] = cos[p, 0]
    want[d // 2] = sin[p, 0]
    assert not np.array_equal(x, want)


def test_rope_preserves_pair_norms():
    d = 128
    cos, sin = okv.rope_tables(4096, d, BASE)
    x = rng_f32(2, 8, 2 * d)
    y = x.copy()
    pos = [0, 1, 7, 100, 1000, 2047, 3000, 4095]
    okv.rope(y, 8, 2, d, pos, cos, sin)
    xp = x.reshape(8, 2, 2, d // 2).astype(np.float64)
    yp = y.reshape(8, 2, 2, d // 2).astype(np.float64)
    nx = np.hypot(xp[:, :, 0], xp[:, :, 1])
    ny = np.hypot(yp[:, :, 0], yp[:, :, 1])
    assert np.max(np.abs(nx - ny) / np.maximum(nx, 1e-6)) < 1e-6


def test_rope_composes_and_depends_on_relative_position():
    """rope(rope(x, a), b) = rope(x, a + b), and <rope(q, m), rope(k, n)> depends on m - n only."""
    d = 64
    cos, sin = okv.rope_tables(1024, d, BASE)
    x = rng_f32(3, d)
    a = x.copy()
    okv.rope(a, 1, 1, d, [100], cos, sin)
    okv.rope(a, 1, 1, d, [250], cos, sin)
    b = x.copy()
    okv.rope(b, 1, 1, d, [350], cos, sin)
    assert np.max(np.abs(a - b)) < 1e-5
    q, k = rng_f32(4, d), rng_f32(5, d)

    def dot(m, n):
        qq, kk = q.copy(), k.copy()
        okv.rope(qq, 1, 1, d, [m], cos, sin)
        okv.rope(kk, 1, 1, d, [n], cos, sin)
        return float(np.dot(qq.astype(np.float64), kk.astype(np.float64)))

    ref = dot(40, 10)
    for t in (1, 17, 300, 900):
        assert abs(dot(40 + t, 10 + t) - ref) < 1e-4


def test_append_kt_is_the_transpose():
    n_ctx, hkv, d, pos, n = 64, 2, 32, 9, 11
    k = rng_f32(6, n, hkv * d)
    kt = np.zeros(hkv * d * n_ctx, np.float32)
    okv.append_kt(kt, n_ctx, hkv, d, pos, k, n)
    cube = kt.reshape(hkv, d, n_ctx)
    assert np.array_equal(cube[:, :, pos:pos + n], np.transpose(k.reshape(n, hkv, d), (1, 2, 0)))
    cube[:, :, pos:pos + n] = 0
    assert not cube.any()  # nothing else written


def test_append_rows_and_llm_step():
    n_ctx, hkv, h, d, n_past, n = 32, 2, 12, 64, 5, 3
    cos, sin = okv.rope_tables(n_ctx, d, BASE)
    q = rng_f32(7, n, h * d)
    k = rng_f32(8, n, hkv * d)
    v = rng_f32(9, n, hkv * d)
    kt = np.zeros(hkv * d * n_ctx, np.float32)
    cv = np.zeros(n_ctx * hkv * d, np.float32)
    q2 = q.copy()
    okv.llm_append(q2, k, v, n, n_past, h, hkv, d, h * d, kt, cv, n_ctx, cos, sin)
    # v rows copied as they are, keys rotated then transposed, q rotated at the same positions
    assert np.array_equal(cv.reshape(n_ctx, -1)[n_past:n_past + n], v)
    assert not cv.reshape(n_ctx, -1)[:n_past].any() and not cv.reshape(n_ctx, -1)[n_past + n:].any()
    kr = k.copy()
    okv.rope(kr, n, hkv, d, range(n_past, n_past + n), cos, sin)
    assert np.array_equal(kt.reshape(hkv, d, n_ctx)[:, :, n_past:n_past + n], np.transpose(kr.reshape(n, hkv, d), (1, 2, 0)))
    qr = q.copy()
    okv.rope(qr, n, h, d, range(n_past, n_past + n), cos, sin)
    assert np.array_equal(q2, qr)
    # a rotated key at position n_past + i differs from the raw key unless the position is 0
    assert not np.array_equal(kr, k)


def test_vectorised_update_matches_line_by_line():
    """llm_append_vec (the timed CPU baseline) against llm_append, bit for bit."""
    n_ctx, hkv, h, d, n_past, n = 96, 2, 12, 128, 40, 9
    cos, sin = okv.rope_tables(n_ctx, d, BASE)
    q, k, v = rng_f32(10, n, h * d), rng_f32(11, n, hkv * d), rng_f32(12, n, hkv * d)
    a_kt, a_v = np.zeros(hkv * d * n_ctx, np.float32), np.zeros(n_ctx * hkv * d, np.float32)
    b_kt, b_v = a_kt.copy(), a_v.copy()
    qa, qb = q.copy(), q.copy()
    okv.llm_append(qa, k, v, n, n_past, h, hkv, d, h * d, a_kt, a_v, n_ctx, cos, sin)
    okv.llm_append_vec(qb, k, v, np.arange(n_past, n_past + n), h, hkv, d, b_kt, b_v, n_ctx, cos, sin)
    assert np.array_equal(qa, qb) and np.array_equal(a_kt, b_kt) and np.array_equal(a_v, b_v)
