"""f64 brute-force attention — TEST INFRASTRUCTURE ONLY (the checker, never the product).

out = softmax(scale * Q K^T + mask) V per head, in float64, with the reference's contract:

* scale is the f32 value 1/sqrt(d) (src/ops.zig:531);
* causal: query i sees keys j <= n_kv - n_q + i (src/ops.zig:466, :534);
* grouped-query attention: head h reads kv head h / (n_head / n_head_kv) (src/ops.zig:476, :521);
* layouts (AttnShape, src/ops.zig:477-492): q [n_q][q_stride], v [n_kv][kv_stride] with head h
  at column h*d; k either [n_kv][kv_stride] (kt_stride 0) or [n_head_kv][d][kt_stride];
* out rows [n_q][out_stride]; only each head's d columns are written (src/ops.zig:540).

This is the same closed form the reference's own test compares against (src/ops.zig:655-704).
"""
from __future__ import annotations

import numpy as np


def _f32_scale(d: int) -> float:
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


def head_views(q, k, v, sh, h):
    """(Q [n_q][d], K [n_kv][d], V [n_kv][d]) of query head h, as float64."""
    d = sh.d
    hk = h // (sh.n_head // sh.n_head_kv)
    qi = np.arange(sh.n_q)[:, None] * sh.q_stride + h * d + np.arange(d)[None, :]
    vi = np.arange(sh.n_kv)[:, None] * sh.kv_stride + hk * d + np.arange(d)[None, :]
    if sh.kt_stride:
        ki = (hk * d + np.arange(d))[None, :] * sh.kt_stride + np.arange(sh.n_kv)[:, None]
    else:
        ki = vi
    q = np.asarray(q).reshape(-1)
    k = np.asarray(k).reshape(-1)
    v = np.asarray(v).reshape(-1)
    return q[qi].astype(np.float64), k[ki].astype(np.float64), v[vi].astype(np.float64)


def attention_heads_f64(q, k, v, sh) -> np.ndarray:
    """Per-head outputs [n_q][n_head][d] in float64."""
    d = sh.d
    out = np.zeros((sh.n_q, sh.n_head, d), dtype=np.float64)
    if sh.n_q == 0 or sh.n_kv == 0:
        return out
    scale = _f32_scale(d)
    i = np.arange(sh.n_q)[:, None]
    j = np.arange(sh.n_kv)[None, :]
    mask = (j > sh.n_kv - sh.n_q + i) if sh.causal else None
    for h in range(sh.n_head):
        Q, K, V = head_views(q, k, v, sh, h)
        s = (Q @ K.T) * scale
        if mask is not None:
            s = np.where(mask, -np.inf, s)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ V
    return out


def attention_f64(q, k, v, sh, out: np.ndarray | None = None) -> np.ndarray:
    """Writes the f64 result into a flat out array laid out [n_q][out_stride] (f64) and returns it."""
    heads = attention_heads_f64(q, k, v, sh)
    n_out = (sh.n_q - 1) * sh.out_stride + sh.n_head * sh.d if sh.n_q else 0
    if out is None:
        out = np.zeros(n_out, dtype=np.float64)
    for i in range(sh.n_q):
        out[i * sh.out_stride: i * sh.out_stride + sh.n_head * sh.d] = heads[i].reshape(-1)
    return out
