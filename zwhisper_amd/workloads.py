"""Seeded synthetic inputs for the attention path and the five benchmark workloads.

The generator is portable and fixed, so a C program, numpy and the tests all draw the same
tensors from a seed:

* SplitMix64: state_i = seed + i * 0x9E3779B97F4A7C15 (i = 1, 2, ...), then the usual
  three-step finaliser (xor-shift 30 / multiply / xor-shift 27 / multiply / xor-shift 31).
* uniform u = (x >> 11) * 2**-53 in [0, 1).
* normals by Box-Muller in f64 over consecutive pairs (u_a, u_b): r = sqrt(-2 ln(1 - u_a)),
  z0 = r cos(2 pi u_b), z1 = r sin(2 pi u_b); cast to f32.

Seeds: base = 0x5A570000 + workload number (1..5); a tensor stream of window or sequence w
uses base + 1000 * w + {lengths: 0, Q: 1, K: 2, V: 3, self-K: 4, self-V: 5}.  K is drawn in
logical [pos][head][d] order and then stored in the layout the call uses, so row-major and
transposed keys hold the same values.  The Qwen2 workloads apply NeoX rotary embedding
(pairs (k, k + d/2), theta 1e6, cos/sin tables computed in f64 and rounded to f32, as
src/llm.zig:128-137 and :221-238) before the values are stored.

This module builds inputs only; it computes no attention.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 started at `seed`, as uint64."""
    seed = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
    i = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = seed + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """n f64 values in [0, 1)."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, n: int) -> np.ndarray:
    """n f32 values, i.i.d. N(0, 1), by Box-Muller over consecutive uniform pairs."""
    pairs = (n + 1) // 2
    u = uniform(seed, 2 * pairs)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
    ang = 2.0 * math.pi * u[1::2]
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(ang)
    z[1::2] = r * np.sin(ang)
    return z[:n].astype(np.float32)


def uniform_centered(seed: int, n: int) -> np.ndarray:
    """n f32 values in [-0.5, 0.5), the distribution of the reference's own attention test."""
    return (uniform(seed, n) - 0.5).astype(np.float32)


def first_u64(seed: int) -> int:
    return int(splitmix64(seed, 1)[0])


def rope_tables(n_pos: int, d: int, theta: float = 1.0e6) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [n_pos][d/2] in f32, computed in f64 (src/llm.zig:128-137)."""
    half = d // 2
    inv = 1.0 / np.power(theta, (2.0 * np.arange(half, dtype=np.float64)) / d)
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def apply_rope(x: np.ndarray, positions: np.ndarray, d: int, theta: float = 1.0e6) -> np.ndarray:
    """NeoX rotary embedding in f32 on x [n][heads][d] at the given positions (src/llm.zig:221-238)."""
    half = d // 2
    pmax = int(positions.max()) + 1 if positions.size else 1
    cos, sin = rope_tables(pmax, d, theta)
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    a = x[..., :half].copy()
    b = x[..., half:].copy()
    out = np.empty_like(x)
    out[..., :half] = a * c - b * s
    out[..., half:] = a * s + b * c
    return out


def seed_base(workload: int) -> int:
    return 0x5A570000 + workload


def stream_seed(workload: int, unit: int, kind: str) -> int:
    off = {"len": 0, "q": 1, "k": 2, "v": 3, "self_k": 4, "self_v": 5}[kind]
    return seed_base(workload) + 1000 * unit + off


def to_kt(k_logical: np.ndarray, kt_stride: int) -> np.ndarray:
    """k [n_kv][n_head_kv][d] -> transposed [n_head_kv][d][kt_stride], zero past n_kv."""
    n_kv, hkv, d = k_logical.shape
    kt = np.zeros((hkv, d, kt_stride), dtype=np.float32)
    kt[:, :, :n_kv] = np.transpose(k_logical, (1, 2, 0))
    return kt


@dataclass
class Workload:
    """One of the five benchmark shapes, with its algorithmic work and its roofline bound."""

    number: int
    name: str
    description: str
    bound: str  # "mfma" or "hbm"
    n_items: int
    n_q: int
    n_head: int
    n_head_kv: int
    d: int
    causal: bool
    kt: bool
    n_kv_cap: int
    extra: dict = field(default_factory=dict)


WORKLOADS = {
    1: Workload(1, "tiny_enc", "Whisper tiny.en encoder self-attention, 1x1500 frames, 6x64, K transposed",
                "mfma", 1, 1500, 6, 6, 64, False, True, 1500),
    2: Workload(2, "base_enc_x16", "Whisper base.en encoder self-attention, 16 windows x 1500 frames, 8x64, "
                "K transposed", "mfma", 16, 1500, 8, 8, 64, False, True, 1500),
    3: Workload(3, "small_dec_x32", "Whisper small.en decoder step, 32 windows: causal self-attention over "
                "n_kv~U[1,448] + cross-attention over 1500, 12x64", "hbm", 32, 1, 12, 12, 64, True, False, 448,
                {"cross_n_kv": 1500}),
    4: Workload(4, "qwen05_prefill", "Qwen2.5-0.5B GQA prefill, 2048 tokens causal, 14q/2kv x 64, "
                "K transposed cache", "mfma", 1, 2048, 14, 2, 64, True, True, 2048),
    5: Workload(5, "qwen15_decode_x64", "Qwen2.5-1.5B GQA decode, 64 sequences n_kv~U[1024,4096], "
                "12q/2kv x 128, K transposed cache", "hbm", 64, 1, 12, 2, 128, True, True, 4096),
}


def kv_lengths(workload: int) -> np.ndarray:
    """Per-item key counts: 1 + r mod 448 (decoder self) or 1024 + r mod 3073 (Qwen decode)."""
    w = WORKLOADS[workload]
    if workload == 3:
        return np.array([1 + first_u64(stream_seed(3, i, "len")) % 448 for i in range(w.n_items)], dtype=np.int64)
    if workload == 5:
        return np.array([1024 + first_u64(stream_seed(5, i, "len")) % 3073 for i in range(w.n_items)],
                        dtype=np.int64)
    return np.full(w.n_items, w.n_kv_cap, dtype=np.int64)


def kt_stride_for(n_kv: int, v: int = 16) -> int:
    """The transposed-key row stride the reference would use: n_kv rounded up to V."""
    return (n_kv + v - 1) // v * v


def algorithmic_work(workload: int, lengths: np.ndarray | None = None) -> float:
    """FLOPs (mfma-bound) or bytes (hbm-bound) of one step of the workload.

    Dense: 4 * d * H * (visible (q, k) pairs), softmax not counted (src/bench.zig:76).
    Decode: K + V read once per KV head (the shared stream), plus Q and O.
    """
    w = WORKLOADS[workload]
    if lengths is None:
        lengths = kv_lengths(workload)
    if w.bound == "mfma":
        if w.causal:
            n = w.n_q
            pairs = n * (n + 1) // 2 + (w.n_kv_cap - n) * n
        else:
            pairs = w.n_q * w.n_kv_cap
        return float(4 * w.d * w.n_head * pairs * w.n_items)
    qo = 2 * w.n_items * w.n_q * w.n_head * w.d * 4
    kv = float(np.sum(2 * lengths.astype(np.float64) * w.n_head_kv * w.d * 4))
    if workload == 3:
        kv += 2 * w.n_items * w.extra["cross_n_kv"] * w.n_head_kv * w.d * 4
        qo *= 2  # a self and a cross call each read Q and write O
    return float(kv + qo)


def make_dense(workload: int, item: int = 0):
    """Inputs of one window/sequence of workload 1, 2 or 4: (q, k_logical, v) as float32.

    q [n_q][H*d]; k_logical [n_kv][Hkv][d]; v [n_kv][Hkv*d].
    """
    w = WORKLOADS[workload]
    n_kv = w.n_kv_cap
    q = normal(stream_seed(workload, item, "q"), w.n_q * w.n_head * w.d).reshape(w.n_q, w.n_head, w.d)
    k = normal(stream_seed(workload, item, "k"), n_kv * w.n_head_kv * w.d).reshape(n_kv, w.n_head_kv, w.d)
    v = normal(stream_seed(workload, item, "v"), n_kv * w.n_head_kv * w.d).reshape(n_kv, w.n_head_kv * w.d)
    if workload == 4:
        pos = np.arange(w.n_q)
        q = apply_rope(q, pos, w.d)
        k = apply_rope(k, np.arange(n_kv), w.d)
    return q.reshape(w.n_q, w.n_head * w.d), k, v


def make_decoder_step(item: int):
    """Workload 3, window `item`: dict of self/cross tensors (row-major, [rows][768])."""
    w = WORKLOADS[3]
    ns = w.n_head * w.d
    n_self = int(kv_lengths(3)[item])
    n_cross = w.extra["cross_n_kv"]
    qq = normal(stream_seed(3, item, "q"), 2 * ns)
    return {
        "q_self": qq[:ns].reshape(1, ns),
        "q_cross": qq[ns:].reshape(1, ns),
        "k_self": normal(stream_seed(3, item, "self_k"), n_self * ns).reshape(n_self, ns),
        "v_self": normal(stream_seed(3, item, "self_v"), n_self * ns).reshape(n_self, ns),
        "k_cross": normal(stream_seed(3, item, "k"), n_cross * ns).reshape(n_cross, ns),
        "v_cross": normal(stream_seed(3, item, "v"), n_cross * ns).reshape(n_cross, ns),
        "n_self": n_self,
    }


def make_llm_decode(item: int):
    """Workload 5, sequence `item`: q [1][H*d] at position n_kv-1, k_logical [n_kv][Hkv][d], v [n_kv][Hkv*d]."""
    w = WORKLOADS[5]
    n_kv = int(kv_lengths(5)[item])
    q = normal(stream_seed(5, item, "q"), w.n_head * w.d).reshape(1, w.n_head, w.d)
    k = normal(stream_seed(5, item, "k"), n_kv * w.n_head_kv * w.d).reshape(n_kv, w.n_head_kv, w.d)
    v = normal(stream_seed(5, item, "v"), n_kv * w.n_head_kv * w.d).reshape(n_kv, w.n_head_kv * w.d)
    q = apply_rope(q, np.array([n_kv - 1]), w.d)
    k = apply_rope(k, np.arange(n_kv), w.d)
    return q.reshape(1, w.n_head * w.d), k, v, n_kv
