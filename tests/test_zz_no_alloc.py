"""zwg_attention_batch_noalloc, the allocation-free entry point, against zwg_attention_batch_dev.

The entry point has no context: its split partials live in the library's static device scratch
(ZWG_NOALLOC_SCRATCH_BYTES per GPU) and it plans as a context with the default workspace does,
so its results must equal the context call's bit for bit (same kernels, same key splits) -- and
both sit within the x3 bar (max abs 5e-5, normwise relative 3e-5) of the f64 closed form.  Each
case runs two calls in a row, the second with a smaller input, so the second call reuses the
scratch the first left behind.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import naive
from zwhisper_amd import workloads as W
from zwhisper_amd.ops import AttnShape

pytestmark = pytest.mark.gpu

TOL_ABS_X3 = 5e-5
TOL_REL_X3 = 3e-5


@pytest.fixture(scope="module")
def torch():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    return torch


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def near_f64(got, ref, what):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    err = float(np.abs(got - ref).max())
    rel = err / max(float(np.abs(ref).max()), 1e-30)
    print(f"{what}: max abs {err:.2e}, normwise rel {rel:.2e}", flush=True)
    assert err <= TOL_ABS_X3 and rel <= TOL_REL_X3, what


def dense_case(seed, n_q, n_kv, h, hkv, d, causal, kt):
    ktw = (n_kv + 7) // 8 * 8 if kt else None
    sh = AttnShape(n_q, n_kv, h, hkv, d, h * d, hkv * d, h * d, causal, ktw)
    q = W.normal(seed, n_q * h * d)
    kl = W.normal(seed + 1, n_kv * hkv * d).reshape(n_kv, hkv, d)
    v = W.normal(seed + 2, n_kv * hkv * d)
    k = W.to_kt(kl, ktw).reshape(-1) if kt else kl.reshape(-1)
    return sh, q, k, v


@pytest.mark.parametrize("mode", [0, 1], ids=["x3", "fp32"])
def test_dense_two_calls_match_the_context_call(torch, mode):
    import zwhisper_amd as z

    # a tiny.en encoder call (keys split 7 ways), then a smaller causal GQA call (split too)
    cases = [dense_case(101, 1500, 1500, 6, 6, 64, False, True), dense_case(111, 300, 420, 8, 2, 64, True, False)]
    with z.Context(0, dense_math=mode) as ctx:
        for i, (sh, q, k, v) in enumerate(cases):
            p = z.plan(sh)
            print(f"case {i}: {sh}, plan chunks {p.max_chunks}, partials {p.workspace_bytes} B", flush=True)
            assert p.max_chunks > 1, "the case must use the scratch"
            qd, kd, vd = dev(torch, q), dev(torch, k), dev(torch, v)
            ref_out = torch.full((sh.out_len(),), 3.0, device="cuda")
            ctx.attention_batch_dev(qd, kd, vd, sh, ref_out, 1, 0, 0, 0, 0)
            out = torch.full((sh.out_len(),), 7.0, device="cuda")
            z.ops.attention_batch_noalloc(qd, kd, vd, sh, out, dense_math=mode)
            torch.cuda.synchronize()
            got, want = out.cpu().numpy(), ref_out.cpu().numpy()
            assert np.array_equal(got, want), f"case {i}: differs from the context call"
            if mode == 0:
                near_f64(got, naive.attention_f64(q, k, v, sh), f"noalloc dense case {i}")


def test_decode_batches_two_calls_on_a_side_stream(torch):
    """Batched decode with per-item key counts (split partials merged from the scratch), on a
    stream of the caller's: 16 sequences, then 5 shorter ones."""
    import zwhisper_amd as z

    cap, h, hkv, d = 2048, 12, 2, 128
    side = torch.cuda.Stream()
    with z.Context(0) as ctx:
        for n, seed in ((16, 201), (5, 301)):
            lengths = (np.arange(n) * 397 % (cap - 64) + 64).astype(np.int32)
            q = W.normal(seed, n * h * d).reshape(n, h * d)
            kl = W.normal(seed + 1, n * cap * hkv * d).reshape(n, cap, hkv, d)
            kt = np.stack([W.to_kt(kl[i], cap) for i in range(n)])
            v = W.normal(seed + 2, n * cap * hkv * d).reshape(n, cap, hkv * d)
            sh = AttnShape(1, cap, h, hkv, d, h * d, hkv * d, h * d, True, cap)
            assert z.plan(sh, n).max_chunks > 1
            qd, kd, vd = dev(torch, q), dev(torch, kt), dev(torch, v)
            nkv = torch.from_numpy(lengths).cuda()
            strides = (h * d, kt[0].size, cap * hkv * d, h * d)
            ref_out = torch.empty(n, h * d, device="cuda")
            ctx.attention_batch_dev(qd, kd, vd, sh, ref_out, n, *strides, nkv)
            torch.cuda.synchronize()
            out = torch.empty(n, h * d, device="cuda")
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                z.ops.attention_batch_noalloc(qd, kd, vd, sh, out, n, *strides, n_kv_dev=nkv, stream=side)
            side.synchronize()
            got = out.cpu().numpy()
            assert np.array_equal(got, ref_out.cpu().numpy()), f"{n} sequences: differs from the context call"
            for i in (0, n - 1):
                L = int(lengths[i])
                shi = AttnShape(1, L, h, hkv, d, h * d, hkv * d, h * d, True, cap)
                near_f64(got[i], naive.attention_f64(q[i], kt[i], v[i], shi), f"noalloc decode seq {i} of {n}")


def test_refuses_a_call_beyond_the_scratch(torch):
    """A call whose split partials exceed the static scratch is refused with a clear error."""
    import zwhisper_amd as z

    sh = AttnShape(2048, 2048, 32, 32, 128, 4096, 4096, 4096, True, None)
    assert z.plan(sh).workspace_bytes > z._lib.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(2048 * 4096, device="cuda")
    with pytest.raises(z.ZwgError, match="static scratch"):
        z.ops.attention_batch_noalloc(x, x, x, sh, x)
