"""CPU restatement of the reference's KV-cache writes — TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's CPU baseline may use this module, as the checker of the device
caches (zwhisper_amd's zwg_kv_*); the product never imports it.

Each function follows the reference line by line, in f32 where the reference computes in f32
(numpy's f32 a*c - b*s rounds each product and the difference, as Zig's default float mode
does; nothing is fused):

* ``rope_tables``  src/llm.zig:128-137  cos/sin [n_ctx][d/2], computed in f64, rounded to f32
* ``rope``         src/llm.zig:221-238  NeoX rotation of (j, j + d/2) pairs, in place
* ``append_rows``  src/decoder.zig:182-183 (K/V projections written into cache rows
                   n_past ..), src/llm.zig:190 (v rows copied into cache_v)
* ``append_kt``    src/llm.zig:185-189  keys scattered into cache_kt[(h*d + p)*n_ctx + col]
* ``llm_append``   src/llm.zig:182-190  the whole per-layer cache update of a forward step

Their checks (closed forms, invariants, a planted mistake) are in tests/test_kv_oracle.py.
"""
from __future__ import annotations

import numpy as np


def rope_tables(n_ctx: int, d: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [n_ctx][d/2]: inv = 1 / base^(2i/d) and ang = p * inv in f64, then f32 (src/llm.zig:131-137)."""
    half = d // 2
    cos = np.empty((n_ctx, half), np.float32)
    sin = np.empty((n_ctx, half), np.float32)
    pos = np.arange(n_ctx, dtype=np.float64)
    for i in range(half):
        inv = 1.0 / np.power(np.float64(base), np.float64(2 * i) / np.float64(d))
        ang = pos * inv
        cos[:, i] = np.cos(ang).astype(np.float32)
        sin[:, i] = np.sin(ang).astype(np.float32)
    return cos, sin


def rope(x: np.ndarray, n: int, heads: int, d: int, positions, cos: np.ndarray, sin: np.ndarray,
         stride: int | None = None) -> None:
    """Rotate rows 0..n-1 of x (row i at position positions[i], `heads` heads of d) in place (src/llm.zig:221-238)."""
    half = d // 2
    stride = heads * d if stride is None else stride
    xf = x.reshape(-1)
    for i in range(n):
        p = int(positions[i])
        c = cos[p]
        s = sin[p]
        for h in range(heads):
            o = i * stride + h * d
            a = xf[o:o + half].copy()
            b = xf[o + half:o + d].copy()
            xf[o:o + half] = a * c - b * s
            xf[o + half:o + d] = a * s + b * c


def append_rows(cache: np.ndarray, kvw: int, pos: int, rows: np.ndarray, n: int) -> None:
    """Rows 0..n-1 of `rows` ([n][kvw]) into cache rows pos .. pos+n-1 ([n_ctx][kvw])."""
    cf = cache.reshape(-1)
    cf[pos * kvw:(pos + n) * kvw] = rows.reshape(-1)[: n * kvw]


def append_kt(cache_kt: np.ndarray, n_ctx: int, n_head_kv: int, d: int, pos: int, k_rows: np.ndarray, n: int) -> None:
    """Keys [n][n_head_kv*d] into the transposed cache: cache_kt[(h*d + p)*n_ctx + pos + i] = k[i][h*d + p]."""
    cf = cache_kt.reshape(-1)
    kf = k_rows.reshape(-1)
    kvw = n_head_kv * d
    for i in range(n):
        col = pos + i
        for h in range(n_head_kv):
            src = kf[i * kvw + h * d:i * kvw + h * d + d]
            for p in range(d):
                cf[(h * d + p) * n_ctx + col] = src[p]


def llm_append(q: np.ndarray | None, k_rows: np.ndarray, v_rows: np.ndarray, n: int, n_past: int, n_head: int,
               n_head_kv: int, d: int, q_stride: int, cache_kt: np.ndarray, cache_v: np.ndarray, n_ctx: int,
               cos: np.ndarray, sin: np.ndarray) -> None:
    """One layer's cache update of a Qwen2 forward step over n new tokens at n_past (src/llm.zig:182-190)."""
    positions = np.arange(n_past, n_past + n)
    if q is not None:
        rope(q, n, n_head, d, positions, cos, sin, stride=q_stride)
    k = k_rows.copy()
    rope(k, n, n_head_kv, d, positions, cos, sin)
    append_kt(cache_kt, n_ctx, n_head_kv, d, n_past, k, n)
    append_rows(cache_v, n_head_kv * d, n_past, v_rows, n)


def llm_append_vec(q: np.ndarray | None, k_rows: np.ndarray, v_rows: np.ndarray, positions: np.ndarray, n_head: int,
                   n_head_kv: int, d: int, cache_kt: np.ndarray, cache_v: np.ndarray, n_ctx: int, cos: np.ndarray,
                   sin: np.ndarray) -> None:
    """``llm_append`` vectorised over tokens, each at its own position (the timed CPU baseline of
    the cache update; it computes the same f32 operations in the same order, so tests require the
    two to agree bit for bit).  q [n][n_head*d], k_rows/v_rows [n][n_head_kv*d]; cache_kt
    [n_head_kv][d][n_ctx], cache_v [n_ctx][n_head_kv*d]."""
    half = d // 2
    positions = np.asarray(positions)
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]

    def rot(x, heads):
        x3 = x.reshape(len(positions), heads, d)
        a = x3[..., :half].copy()
        b = x3[..., half:].copy()
        x3[..., :half] = a * c - b * s
        x3[..., half:] = a * s + b * c

    if q is not None:
        rot(q, n_head)
    k = k_rows.copy()
    rot(k, n_head_kv)
    kt = cache_kt.reshape(n_head_kv * d, n_ctx)
    kt[:, positions] = k.reshape(len(positions), n_head_kv * d).T
    cache_v.reshape(n_ctx, n_head_kv * d)[positions] = v_rows.reshape(len(positions), n_head_kv * d)
