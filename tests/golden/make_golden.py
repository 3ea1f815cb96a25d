"""Writes tests/golden/attn_golden.npz: small attention cases with f64 expected outputs.

    python tests/golden/make_golden.py

The reference holds no golden vectors for attention: its only check is a comparison with a
naive triple loop (src/ops.zig:655-704).  These fixtures are that closed form, evaluated in
float64 (oracle/naive.py), on seeded inputs (zwhisper_amd/workloads.py), one case per caller
family: encoder (row-major and transposed K), decoder self/cross at n_q = 1, decoder prompt,
Qwen2 GQA prefill and decode over a transposed cache, BERT's d = 32, strided rows, and the
reference test's own shape.  Small cases store their inputs as arrays; the larger ones store
their seeds plus a SHA-256 of the regenerated inputs, which the loader checks.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import naive  # noqa: E402
from zwhisper_amd import workloads as W  # noqa: E402
from zwhisper_amd.ops import AttnShape  # noqa: E402

OUT = os.path.join(HERE, "attn_golden.npz")


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a, dtype=np.float32).tobytes())
    return h.hexdigest()


def gen_inputs(case: dict):
    """q, k (stored layout), v flat float32 arrays for a case description."""
    sh: AttnShape = case["shape"]
    seed = case["seed"]
    dist = W.uniform_centered if case.get("dist") == "uniform" else W.normal
    n_rows_q = sh.n_q
    q = np.zeros(max(sh.q_len(), 1), dtype=np.float32)
    qv = dist(seed + 1, n_rows_q * sh.n_head * sh.d).reshape(n_rows_q, sh.n_head * sh.d)
    for i in range(n_rows_q):
        q[i * sh.q_stride: i * sh.q_stride + sh.n_head * sh.d] = qv[i]
    kl = dist(seed + 2, sh.n_kv * sh.n_head_kv * sh.d).reshape(sh.n_kv, sh.n_head_kv, sh.d)
    vv = dist(seed + 3, sh.n_kv * sh.n_head_kv * sh.d).reshape(sh.n_kv, sh.n_head_kv * sh.d)
    if case.get("rope"):
        qv3 = q[: sh.q_len()].copy()
        rows = np.stack([qv3[i * sh.q_stride: i * sh.q_stride + sh.n_head * sh.d] for i in range(n_rows_q)])
        rows = W.apply_rope(rows.reshape(n_rows_q, sh.n_head, sh.d), np.arange(sh.n_kv - sh.n_q, sh.n_kv), sh.d)
        for i in range(n_rows_q):
            q[i * sh.q_stride: i * sh.q_stride + sh.n_head * sh.d] = rows[i].reshape(-1)
        kl = W.apply_rope(kl, np.arange(sh.n_kv), sh.d)
    if sh.kt_stride:
        # as much of the [hkv][d][kt_stride] cache as the reference reads: round_up(n_kv, V)
        # columns of the last row (src/ops.zig:529-530)
        k = W.to_kt(kl, sh.kt_stride).reshape(-1)
        k = np.ascontiguousarray(k[: (sh.n_head_kv * sh.d - 1) * sh.kt_stride + (sh.n_kv + 15) // 16 * 16])
    else:
        k = np.zeros(max(sh.k_len(), 1), dtype=np.float32)
        for t in range(sh.n_kv):
            k[t * sh.kv_stride: t * sh.kv_stride + sh.n_head_kv * sh.d] = kl[t].reshape(-1)
    v = np.zeros(max(sh.v_len(), 1), dtype=np.float32)
    for t in range(sh.n_kv):
        v[t * sh.kv_stride: t * sh.kv_stride + sh.n_head_kv * sh.d] = vv[t]
    return q, k, v


def S(n_q, n_kv, h, hkv, d, causal, kt=None, qs=None, kvs=None, os_=None):
    return AttnShape(n_q, n_kv, h, hkv, d, qs or h * d, kvs or hkv * d, os_ or h * d, causal, kt)


# name, shape, seed, extras
CASES = [
    ("ref_test_noncausal", S(70, 90, 2, 2, 32, False), 900, {"dist": "uniform"}),
    ("ref_test_causal", S(70, 90, 2, 2, 32, True), 900, {"dist": "uniform"}),
    ("dec_self_nkv1", S(1, 1, 12, 12, 64, True), 910, {}),
    ("dec_self_nkv17", S(1, 17, 12, 12, 64, True), 920, {}),
    ("dec_self_nkv448", S(1, 448, 2, 2, 64, True), 930, {}),
    ("dec_cross_nkv1500", S(1, 1500, 1, 1, 64, False), 940, {"store": "seed"}),
    ("dec_prompt_causal", S(5, 12, 6, 6, 64, True), 950, {}),
    ("enc_rowmajor", S(200, 200, 2, 2, 64, False), 960, {}),
    ("enc_kt", S(200, 200, 2, 2, 64, False, kt=208), 970, {"store": "seed"}),
    ("gqa_prefill_kt", S(150, 150, 7, 1, 64, True, kt=160), 980, {"rope": True, "store": "seed"}),
    ("gqa_chunk_kt", S(7, 40, 14, 2, 64, True, kt=48), 990, {"rope": True}),
    ("gqa_decode_kt_d128", S(1, 300, 12, 2, 128, True, kt=320), 1000, {"rope": True, "store": "seed"}),
    ("gqa_decode_rows8", S(4, 33, 4, 2, 64, True), 1010, {}),
    ("bert_d32", S(20, 20, 12, 12, 32, False), 1020, {}),
    ("strided_rows", S(33, 47, 2, 2, 32, False, qs=96, kvs=80, os_=72), 1030, {}),
    ("flash_d128_rowmajor", S(130, 177, 3, 1, 128, True, kvs=132), 1040, {"store": "seed"}),
    ("nkv0", S(3, 0, 2, 2, 64, False), 1050, {}),
    ("decode_long_kt_4096", S(1, 4096, 6, 1, 128, True, kt=4096), 1060, {"rope": True, "store": "seed"}),
]


def main() -> None:
    data: dict[str, np.ndarray] = {}
    names = []
    for name, sh, seed, extra in CASES:
        case = {"shape": sh, "seed": seed, **extra}
        q, k, v = gen_inputs(case)
        out = naive.attention_f64(q, k, v, sh)
        names.append(name)
        data[f"{name}/shape"] = np.array([sh.n_q, sh.n_kv, sh.n_head, sh.n_head_kv, sh.d, sh.q_stride, sh.kv_stride,
                                          sh.out_stride, sh.kt_stride or 0, int(sh.causal)], dtype=np.int64)
        data[f"{name}/seed"] = np.array([seed], dtype=np.int64)
        data[f"{name}/flags"] = np.array([int(extra.get("dist") == "uniform"), int(bool(extra.get("rope")))],
                                         dtype=np.int64)
        data[f"{name}/expected"] = out
        data[f"{name}/sha256"] = np.array(digest(q, k, v))
        if extra.get("store") != "seed":
            data[f"{name}/q"], data[f"{name}/k"], data[f"{name}/v"] = q, k, v
    data["names"] = np.array(names)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}: {len(names)} cases, {os.path.getsize(OUT) / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
