"""GPU parity for head dims without kernels of their own.

The reference takes any head dim d with d % V == 0 (src/ops.zig:564).  This build's kernels are
built for d = 32, 64 and 128; any other d % 4 == 0 up to 128 runs on the kernels of the next of
them over zero-padded copies of q, k, v and out (zwhisper_amd/csrc/attn_pad.hip).  Each case is
checked against the f64 closed form (oracle/naive.py) at the bars of tests/test_gpu_parity.py:
the x3 bar (max abs 5e-5, normwise relative 3e-5) for dense calls of an x3 context, the f32 bar
(2e-4, 1e-3) otherwise.  Covered: the dense kernel in both modes with row-major and transposed
keys, causal GQA and non-causal; the decode kernels over row-major and transposed caches with
per-item key counts; output columns outside each head's d left untouched; the allocation-free
entry point's refusal of such d.  Head dims above 128 (up to 1024) run on a plain f32 kernel
(zwhisper_amd/csrc/attn_generic.hip) in either dense mode, held to the f32 bar: dense and decode
shapes, row-major and transposed keys, per-item key counts, the host drop-in and the
allocation-free entry point (which needs no padded copies for them).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {True: (5e-5, 3e-5), False: (2e-4, 1e-3)}  # x3 dense, f32
SENTINEL = 7.25
DIMS = [4, 16, 24, 48, 80, 100, 112]


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


def make(rng, n_q, n_kv, h, hk, d, kt, pad=4):
    """q, k (row-major or transposed), v as flat f32 arrays, and the shape; strides carry `pad`
    extra columns so the calls see gaps."""
    from zwhisper_amd.ops import AttnShape

    qs, kvs, os_ = h * d + pad, hk * d + pad, h * d + pad
    q = rng.standard_normal((n_q, qs)).astype(np.float32)
    kl = rng.standard_normal((n_kv, hk, d)).astype(np.float32)
    v = rng.standard_normal((n_kv, kvs)).astype(np.float32)
    if kt:
        kts = (n_kv + 3) // 4 * 4 + 4
        k = np.zeros((hk, d, kts), np.float32)
        k[:, :, :n_kv] = np.transpose(kl, (1, 2, 0))
    else:
        kts = None
        k = rng.standard_normal((n_kv, kvs)).astype(np.float32)
        k[:, : hk * d] = kl.reshape(n_kv, hk * d)
    return q.reshape(-1), k.reshape(-1), v.reshape(-1), (qs, kvs, os_, kts)


def check(got, q, k, v, sh, x3, what):
    from oracle import naive

    ref = naive.attention_heads_f64(q, k, v, sh).reshape(sh.n_q, sh.n_head * sh.d)
    got2 = got.reshape(sh.n_q, sh.out_stride)
    # the columns past n_head * d of every row keep the caller's contents
    assert np.all(got2[:, sh.n_head * sh.d:] == np.float32(SENTINEL)), f"{what}: wrote outside the heads"
    out = got2[:, : sh.n_head * sh.d].astype(np.float64)
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    err = float(np.abs(out - ref).max()) if ref.size else 0.0
    rel = err / max(float(np.abs(ref).max()) if ref.size else 0.0, 1e-30)
    ta, tr = TOL[x3]
    print(f"{what}: max abs {err:.2e} rel {rel:.2e}")
    assert err <= ta and rel <= tr, f"{what}: max abs {err:.3e} rel {rel:.3e}"


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("kind", ["enc_rowmajor", "enc_kt", "prefill_gqa_kt", "decode_rowmajor", "decode_gqa_kt"])
def test_head_dim_single(torch, ctx, d, kind):
    import zwhisper_amd as z
    from zwhisper_amd.ops import AttnShape

    rng = np.random.default_rng(1000 + d)
    n_q, n_kv, h, hk, causal, kt = {
        "enc_rowmajor": (150, 170, 4, 4, False, False),
        "enc_kt": (150, 170, 3, 3, False, True),
        "prefill_gqa_kt": (200, 260, 6, 2, True, True),
        "decode_rowmajor": (1, 700, 8, 8, True, False),
        "decode_gqa_kt": (1, 900, 8, 2, True, True),
    }[kind]
    q, k, v, (qs, kvs, os_, kts) = make(rng, n_q, n_kv, h, hk, d, kt)
    sh = AttnShape(n_q, n_kv, h, hk, d, qs, kvs, os_, causal, kts)
    dense = z.plan(sh).kernel == 1
    out = torch.full((n_q * os_,), SENTINEL, dtype=torch.float32, device="cuda")
    ctx.attention_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh, out)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), q, k, v, sh, dense and ctx.mode == "x3", f"{kind} d={d} {ctx.mode}")


@pytest.mark.parametrize("d", [24, 80])
@pytest.mark.parametrize("kt", [False, True])
def test_head_dim_batch_per_item_lengths(torch, ctx, d, kt):
    """A batch of decode steps with their own key counts (0 included) at a padded head dim."""
    from zwhisper_amd.ops import AttnShape

    rng = np.random.default_rng(77 + d)
    n_items, cap, h, hk = 5, 600, 12, 2
    lengths = np.array([1, 37, 255, 600, 0], np.int32)
    items = [make(rng, 1, cap, h, hk, d, kt) for _ in range(n_items)]
    qs, kvs, os_, kts = items[0][3]
    sh = AttnShape(1, cap, h, hk, d, qs, kvs, os_, True, kts)
    q = np.stack([it[0] for it in items])
    k = np.stack([it[1] for it in items])
    v = np.stack([it[2] for it in items])
    out = torch.full((n_items, os_), SENTINEL, dtype=torch.float32, device="cuda")
    nkv = torch.from_numpy(lengths).cuda()
    ctx.attention_batch_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh,
                            out, n_items, q[0].size, k[0].size, v[0].size, os_, nkv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, L in enumerate(lengths):
        shi = AttnShape(1, int(L), h, hk, d, qs, kvs, os_, True, kts)
        if L == 0:
            # no keys: the kernels write zeros, as the reference's empty softmax sum gives nothing
            assert np.all(got[i, : h * d] == 0.0) and np.all(got[i, h * d:] == np.float32(SENTINEL))
            continue
        check(got[i], q[i], k[i], v[i], shi, False, f"item {i} n_kv={L} d={d} kt={kt} {ctx.mode}")


def test_head_dim_host_dropin(torch, ctx):
    """zwg_attention_ex with host buffers at d = 48 (the padded copies live in the context)."""
    from zwhisper_amd.ops import AttnShape

    rng = np.random.default_rng(5)
    q, k, v, (qs, kvs, os_, kts) = make(rng, 90, 120, 4, 2, 48, True)
    sh = AttnShape(90, 120, 4, 2, 48, qs, kvs, os_, True, kts)
    out = np.full(90 * os_, SENTINEL, np.float32)
    ctx.attention_ex_host(q, k, v, sh, out)
    check(out, q, k, v, sh, ctx.mode == "x3", f"host drop-in d=48 {ctx.mode}")


def test_head_dim_noalloc_refused(torch):
    import zwhisper_amd as z
    from zwhisper_amd.ops import AttnShape

    sh = AttnShape(4, 8, 2, 2, 48, 96, 96, 96, False, None)
    t = torch.zeros(4096, device="cuda")
    with pytest.raises(z.ZwgError, match="head dims other than 32, 64 and 128"):
        z.ops.attention_batch_noalloc(t, t, t, sh, t)


BIG_DIMS = [132, 192, 256, 516, 1024]


@pytest.mark.parametrize("d", BIG_DIMS)
@pytest.mark.parametrize("kind", ["enc_rowmajor", "enc_kt", "prefill_gqa_kt", "decode_rowmajor", "decode_gqa_kt"])
def test_head_dim_above_128(torch, d, kind):
    import zwhisper_amd as z
    from zwhisper_amd.ops import AttnShape

    rng = np.random.default_rng(3000 + d)
    n_q, n_kv, h, hk, causal, kt = {
        "enc_rowmajor": (70, 130, 3, 3, False, False),
        "enc_kt": (70, 130, 2, 2, False, True),
        "prefill_gqa_kt": (90, 150, 6, 2, True, True),
        "decode_rowmajor": (1, 333, 4, 4, True, False),
        "decode_gqa_kt": (1, 400, 8, 2, True, True),
    }[kind]
    q, k, v, (qs, kvs, os_, kts) = make(rng, n_q, n_kv, h, hk, d, kt)
    sh = AttnShape(n_q, n_kv, h, hk, d, qs, kvs, os_, causal, kts)
    assert z.plan(sh).kernel == 3
    with z.Context(0) as c:
        out = torch.full((n_q * os_,), SENTINEL, dtype=torch.float32, device="cuda")
        c.attention_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh, out)
        torch.cuda.synchronize()
    check(out.cpu().numpy(), q, k, v, sh, False, f"{kind} d={d}")


@pytest.mark.parametrize("kt", [False, True])
def test_head_dim_above_128_batch_per_item_lengths(torch, kt):
    """A batch of decode steps with their own key counts (0 included) at d = 256."""
    import zwhisper_amd as z
    from zwhisper_amd.ops import AttnShape

    d = 256
    rng = np.random.default_rng(99)
    n_items, cap, h, hk = 4, 300, 4, 2
    lengths = np.array([1, 77, 300, 0], np.int32)
    items = [make(rng, 1, cap, h, hk, d, kt) for _ in range(n_items)]
    qs, kvs, os_, kts = items[0][3]
    sh = AttnShape(1, cap, h, hk, d, qs, kvs, os_, True, kts)
    q = np.stack([it[0] for it in items])
    k = np.stack([it[1] for it in items])
    v = np.stack([it[2] for it in items])
    with z.Context(0) as c:
        out = torch.full((n_items, os_), SENTINEL, dtype=torch.float32, device="cuda")
        c.attention_batch_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh,
                              out, n_items, q[0].size, k[0].size, v[0].size, os_, torch.from_numpy(lengths).cuda())
        torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, L in enumerate(lengths):
        shi = AttnShape(1, int(L), h, hk, d, qs, kvs, os_, True, kts)
        if L == 0:
            assert np.all(got[i, : h * d] == 0.0) and np.all(got[i, h * d:] == np.float32(SENTINEL))
            continue
        check(got[i], q[i], k[i], v[i], shi, False, f"item {i} n_kv={L} d={d} kt={kt}")


def test_head_dim_above_128_dropin_and_noalloc(torch):
    """d = 192 through the host drop-in, and through the allocation-free entry point, which needs
    no padded copies for head dims above 128."""
    import zwhisper_amd as z
    from zwhisper_amd.ops import AttnShape

    rng = np.random.default_rng(7)
    q, k, v, (qs, kvs, os_, kts) = make(rng, 50, 80, 4, 2, 192, False)
    sh = AttnShape(50, 80, 4, 2, 192, qs, kvs, os_, True, kts)
    out = np.full(50 * os_, SENTINEL, np.float32)
    with z.Context(0) as c:
        c.attention_ex_host(q, k, v, sh, out)
    check(out, q, k, v, sh, False, "host drop-in d=192")
    dev_out = torch.full((50 * os_,), SENTINEL, dtype=torch.float32, device="cuda")
    z.ops.attention_batch_noalloc(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                  sh, dev_out)
    torch.cuda.synchronize()
    assert np.array_equal(dev_out.cpu().numpy(), out), "the allocation-free entry point differs from the drop-in"
