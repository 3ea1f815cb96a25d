"""GPU parity over seeded random shapes: every path of the attention entry point at once.

Each case draws a batch size, KV heads and GQA group, head dim (built and padded dims), causal or
not, row-major or transposed K, query and key counts (n_q = 1 takes the decode kernels), strides
with padding columns, and per-item key counts (some 0 for decode; at least n_q for causal dense
calls).  Every item's output is checked against the f64 closed form (oracle/naive.py) at the bar
of the arithmetic that ran -- the x3 bar (max abs 5e-5, normwise relative 3e-5) for dense calls of
an x3 context, the f32 bar (2e-4, 1e-3) otherwise -- and the padding columns of `out` must keep
their contents.  Both dense modes run every case.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SENTINEL = -3.5
N_CASES = 200


@pytest.fixture(scope="module")
def torch():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    return torch


@pytest.fixture(scope="module", params=["x3", "fp32"])
def ctx(request, torch):
    import zwhisper_amd as z

    c = z.Context(0, dense_math=z.DENSE_X3 if request.param == "x3" else z.DENSE_FP32)
    c.mode = request.param
    yield c
    c.close()


def draw(seed: int):
    rng = np.random.default_rng(seed)
    hkv = int(rng.choice([1, 2, 3, 4]))
    group = int(rng.choice([1, 2, 3, 4, 7]))
    h = hkv * group
    d = int(rng.choice([16, 32, 48, 64, 96, 128]))
    causal = bool(rng.integers(2))
    kt = bool(rng.integers(2))
    decode = rng.random() < 0.35
    n_q = 1 if decode else int(rng.choice([2, 3, 7, 33, 64, 129, 300]))
    n_kv = n_q + int(rng.integers(0, 700)) if causal else int(rng.integers(1, 900))
    n_batch = int(rng.choice([1, 2, 3, 5]))
    per_item = n_batch > 1 and rng.random() < 0.6
    lo = n_q if causal else 0
    lengths = [int(rng.integers(lo, n_kv + 1)) for _ in range(n_batch)] if per_item else [n_kv] * n_batch
    pad = [4 * int(rng.integers(0, 3)) for _ in range(4)]
    return dict(rng=rng, h=h, hkv=hkv, d=d, causal=causal, kt=kt, n_q=n_q, n_kv=n_kv, n_batch=n_batch,
                per_item=per_item, lengths=lengths, pad=pad)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_fuzz_shape(torch, ctx, seed):
    import zwhisper_amd as z
    from oracle import naive
    from zwhisper_amd.ops import AttnShape

    c = draw(7000 + seed)
    rng, h, hkv, d, n_q, n_kv, B = c["rng"], c["h"], c["hkv"], c["d"], c["n_q"], c["n_kv"], c["n_batch"]
    qs, kvs, os_ = h * d + c["pad"][0], hkv * d + c["pad"][1], h * d + c["pad"][2]
    kts = ((n_kv + 3) // 4 * 4 + c["pad"][3]) if c["kt"] else None
    sh = AttnShape(n_q, n_kv, h, hkv, d, qs, kvs, os_, c["causal"], kts)
    print(f"case {seed}: {sh} batch {B} lengths {c['lengths']} mode {ctx.mode}", flush=True)
    q = rng.standard_normal((B, n_q, qs)).astype(np.float32)
    v = rng.standard_normal((B, n_kv, kvs)).astype(np.float32)
    kl = rng.standard_normal((B, n_kv, hkv, d)).astype(np.float32)
    if c["kt"]:
        k = np.zeros((B, hkv, d, kts), np.float32)
        k[..., :n_kv] = np.transpose(kl, (0, 2, 3, 1))
    else:
        k = rng.standard_normal((B, n_kv, kvs)).astype(np.float32)
        k[:, :, : hkv * d] = kl.reshape(B, n_kv, hkv * d)
    out = torch.full((B, n_q, os_), SENTINEL, dtype=torch.float32, device="cuda")
    nkv = torch.tensor(c["lengths"], dtype=torch.int32, device="cuda") if c["per_item"] else None
    ctx.attention_batch_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh,
                            out, B, q[0].size, k[0].size, v[0].size, n_q * os_, nkv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    dense = z.plan(sh, B).kernel == 1
    tol_abs, tol_rel = (5e-5, 3e-5) if dense and ctx.mode == "x3" else (2e-4, 1e-3)
    for i, L in enumerate(c["lengths"]):
        assert np.all(got[i][:, h * d:] == np.float32(SENTINEL)), f"item {i}: wrote outside the heads"
        res = got[i][:, : h * d].astype(np.float64)
        assert np.all(np.isfinite(res)), f"item {i}: non-finite output"
        if L == 0:
            assert np.all(res == 0.0), f"item {i}: no keys must give zeros"
            continue
        shi = AttnShape(n_q, L, h, hkv, d, qs, kvs, os_, c["causal"], kts)
        ref = naive.attention_heads_f64(q[i].reshape(-1), k[i].reshape(-1), v[i].reshape(-1), shi).reshape(n_q, h * d)
        err = float(np.abs(res - ref).max())
        rel = err / max(float(np.abs(ref).max()), 1e-30)
        assert err <= tol_abs and rel <= tol_rel, f"item {i} (n_kv {L}): max abs {err:.3e} rel {rel:.3e}"
