"""GPU parity at the benchmark workloads' full sizes, and the batch/stream/split paths.

Each workload is checked against the f64 closed form (oracle/naive.py) on the same seeded
inputs the benchmark uses.  Bars (include/zw_gpu.h): a context in the x3 dense mode (the
default) is held to max abs error <= 5e-5 and normwise relative error ||gpu - ref||_inf /
||ref||_inf <= 3e-5 for every call; the fp32 dense mode to the reference's f32 bar, 2e-4 and
1e-3.  The dense workloads run in both modes.  Where a full f64 reference of every item would be slow,
some items are compared directly and the rest through properties that hold at any size:
each output lies in the per-dimension hull of the visible value rows, and a batched call agrees
with per-item calls.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import naive
from zwhisper_amd import workloads as W
from zwhisper_amd.ops import AttnShape

pytestmark = pytest.mark.gpu

TOL_ABS = 2e-4  # f32 bar
TOL_REL = 1e-3
TOL_ABS_X3 = 5e-5  # x3 dense mode
TOL_REL_X3 = 3e-5
MODES = ["x3", "fp32"]


@pytest.fixture(scope="module")
def torch():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    return torch


@pytest.fixture(scope="module")
def ctx(torch):
    import zwhisper_amd as z

    c = z.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def ctx_fp32(torch):
    import zwhisper_amd as z

    c = z.Context(0, dense_math=z.DENSE_FP32)
    yield c
    c.close()


def check(got, ref, what, x3: bool = True, v_scale: float = 1.0):
    """Max abs and normwise relative error against ref, to the x3 bar (x3=True) or the f32 bar.
    The absolute bars hold for values of order one; an output row is a weighted mean of value
    rows, so for values up to v_scale in magnitude the absolute bar scales by v_scale."""
    tol_abs, tol_rel = (TOL_ABS_X3, TOL_REL_X3) if x3 else (TOL_ABS, TOL_REL)
    tol_abs *= max(v_scale, 1.0)
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = float(np.abs(got - ref).max())
    rel = err / max(float(np.abs(ref).max()), 1e-30)
    print(f"{what}: max abs {err:.2e}, normwise rel {rel:.2e}", flush=True)
    assert err <= tol_abs and rel <= tol_rel, f"{what}: max abs {err:.3e} (<= {tol_abs}), rel {rel:.3e} (<= {tol_rel})"


def mode_ctx(request, mode):
    return request.getfixturevalue("ctx" if mode == "x3" else "ctx_fp32")


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


@pytest.mark.parametrize("mode", MODES)
def test_tiny_encoder_full(torch, request, mode):
    """Workload 1: 1500 x 1500, 6 heads x 64, transposed K (kt_stride 1504), both dense modes."""
    ctx = mode_ctx(request, mode)
    w = W.WORKLOADS[1]
    q, kl, v = W.make_dense(1, 0)
    sh = AttnShape(1500, 1500, 6, 6, 64, 384, 384, 384, False, 1504)
    kt = W.to_kt(kl, 1504)
    out = torch.empty(1500 * 384, device="cuda")
    ctx.attention_dev(dev(torch, q), dev(torch, kt), dev(torch, v), sh, out)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), naive.attention_f64(q, kt, v, sh), f"{w.name} ({mode})", x3=mode == "x3")


@pytest.mark.parametrize("mode", MODES)
def test_base_encoder_batch(torch, request, mode):
    """Workload 2: 16 windows in one batched call; windows 0 and 15 against f64, all windows
    against per-window calls; both dense modes."""
    ctx = mode_ctx(request, mode)
    w = W.WORKLOADS[2]
    sh = AttnShape(1500, 1500, 8, 8, 64, 512, 512, 512, False, 1504)
    qs, kts, vs = [], [], []
    for i in range(16):
        q, kl, v = W.make_dense(2, i)
        qs.append(q)
        kts.append(W.to_kt(kl, 1504))
        vs.append(v)
    q, kt, v = dev(torch, np.stack(qs)), dev(torch, np.stack(kts)), dev(torch, np.stack(vs))
    out = torch.empty(16, 1500, 512, device="cuda")
    ctx.attention_batch_dev(q, kt, v, sh, out, 16, 1500 * 512, 8 * 64 * 1504, 1500 * 512, 1500 * 512)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i in (0, 15):
        check(got[i], naive.attention_f64(qs[i], kts[i], vs[i], sh), f"{w.name} window {i} ({mode})", x3=mode == "x3")
    one = torch.empty(1500, 512, device="cuda")
    for i in range(16):
        ctx.attention_dev(q[i], kt[i], v[i], sh, one)
        torch.cuda.synchronize()
        assert np.max(np.abs(one.cpu().numpy() - got[i])) <= 1e-5, f"window {i}: batch != single call"


def test_decoder_step_all_windows(torch, ctx):
    """Workload 3: 32 windows, causal self-attention over per-window cache lengths (device
    int32 array) plus cross-attention over 1500 frames, every window against f64."""
    w = W.WORKLOADS[3]
    ns, cap = 768, 448
    lengths = W.kv_lengths(3)
    qs = np.zeros((32, ns), np.float32)
    qc = np.zeros((32, ns), np.float32)
    ks = np.zeros((32, cap, ns), np.float32)
    vs = np.zeros((32, cap, ns), np.float32)
    kc = np.zeros((32, 1500, ns), np.float32)
    vc = np.zeros((32, 1500, ns), np.float32)
    steps = [W.make_decoder_step(i) for i in range(32)]
    for i, s in enumerate(steps):
        qs[i], qc[i] = s["q_self"][0], s["q_cross"][0]
        ks[i, : s["n_self"]], vs[i, : s["n_self"]] = s["k_self"], s["v_self"]
        kc[i], vc[i] = s["k_cross"], s["v_cross"]
    nkv = torch.from_numpy(lengths.astype(np.int32)).cuda()
    o_self = torch.empty(32, ns, device="cuda")
    o_cross = torch.empty(32, ns, device="cuda")
    sh_self = AttnShape(1, cap, 12, 12, 64, ns, ns, ns, True)
    sh_cross = AttnShape(1, 1500, 12, 12, 64, ns, ns, ns, False)
    ctx.attention_batch_dev(dev(torch, qs), dev(torch, ks), dev(torch, vs), sh_self, o_self, 32, ns, cap * ns,
                            cap * ns, ns, nkv)
    ctx.attention_batch_dev(dev(torch, qc), dev(torch, kc), dev(torch, vc), sh_cross, o_cross, 32, ns, 1500 * ns,
                            1500 * ns, ns)
    torch.cuda.synchronize()
    gs, gc = o_self.cpu().numpy(), o_cross.cpu().numpy()
    for i, s in enumerate(steps):
        n = s["n_self"]
        ref_s = naive.attention_f64(s["q_self"], s["k_self"], s["v_self"], AttnShape(1, n, 12, 12, 64, ns, ns, ns, True))
        check(gs[i], ref_s, f"{w.name} self window {i} (n_kv {n})")
        check(gc[i], naive.attention_f64(s["q_cross"], s["k_cross"], s["v_cross"], sh_cross),
              f"{w.name} cross window {i}")


@pytest.mark.parametrize("mode", MODES)
def test_qwen_prefill_full(torch, request, mode):
    """Workload 4: 2048 tokens causal, 14 query / 2 KV heads, transposed cache of 2048 columns,
    both dense modes."""
    ctx = mode_ctx(request, mode)
    w = W.WORKLOADS[4]
    q, kl, v = W.make_dense(4, 0)
    kt = W.to_kt(kl, 2048)
    sh = AttnShape(2048, 2048, 14, 2, 64, 896, 128, 896, True, 2048)
    out = torch.empty(2048 * 896, device="cuda")
    ctx.attention_dev(dev(torch, q), dev(torch, kt), dev(torch, v), sh, out)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), naive.attention_f64(q, kt, v, sh), f"{w.name} ({mode})", x3=mode == "x3")


@pytest.mark.parametrize("mode", ["x3", "fp32"])
def test_qwen_prefill_as_llm_prompt(torch, request, mode):
    """Workload 4 as llm.prompt feeds it (src/llm.zig:258-266): 8 calls of 256 rows, call i with the
    cache's first 256 (i + 1) keys (transposed cache of 2048 columns), rows written into one
    output; the result is the one-call prefill's, checked against f64."""
    ctx = mode_ctx(request, mode)
    q, kl, v = W.make_dense(4, 0)
    kt = W.to_kt(kl, 2048)
    qd, kd, vd = dev(torch, q), dev(torch, kt), dev(torch, v)
    out = torch.full((2048, 896), float("nan"), device="cuda")
    for i in range(8):
        sh = AttnShape(256, 256 * (i + 1), 14, 2, 64, 896, 128, 896, True, 2048)
        ctx.attention_dev(qd.view(2048, 896)[256 * i: 256 * (i + 1)], kd, vd, sh, out[256 * i: 256 * (i + 1)])
    torch.cuda.synchronize()
    full = AttnShape(2048, 2048, 14, 2, 64, 896, 128, 896, True, 2048)
    check(out.cpu().numpy().reshape(-1), naive.attention_f64(q, kt, v, full), f"prefill 8 x 256 ({mode})",
          x3=mode == "x3")


def test_qwen_decode_all_sequences(torch, ctx):
    """Workload 5: 64 sequences with cache lengths 1024..4096, 12/2 heads x 128, one batched call."""
    w = W.WORKLOADS[5]
    cap = 4096
    q = np.zeros((64, 1536), np.float32)
    kt = np.zeros((64, 2, 128, cap), np.float32)
    v = np.zeros((64, cap, 256), np.float32)
    items = []
    for i in range(64):
        qi, kl, vi, n = W.make_llm_decode(i)
        q[i], kt[i], v[i, :n] = qi[0], W.to_kt(kl, cap), vi
        items.append((qi, kt[i].copy(), vi, n))
    nkv = torch.from_numpy(W.kv_lengths(5).astype(np.int32)).cuda()
    out = torch.empty(64, 1536, device="cuda")
    sh = AttnShape(1, cap, 12, 2, 128, 1536, 256, 1536, True, cap)
    ctx.attention_batch_dev(dev(torch, q), dev(torch, kt), dev(torch, v), sh, out, 64, 1536, 2 * 128 * cap,
                            cap * 256, 1536, nkv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, (qi, kti, vi, n) in enumerate(items):
        ref = naive.attention_f64(qi, kti, vi, AttnShape(1, n, 12, 2, 128, 1536, 256, 1536, True, cap))
        check(got[i], ref, f"{w.name} sequence {i} (n_kv {n})")


@pytest.mark.parametrize("kt", [False, True])
def test_ragged_lengths_edge_cases(torch, ctx, kt):
    """Per-item cache lengths at the edges: 1, 2, 3, 255, 256, 257, not multiples of 4, capacity."""
    lengths = [1, 2, 3, 5, 255, 256, 257, 511, 1023, 1500]
    cap, h, hkv, d = 1504, 4, 2, 64
    n = len(lengths)
    q = W.normal(11, n * h * d).reshape(n, h * d)
    kl = W.normal(12, n * cap * hkv * d).reshape(n, cap, hkv, d)
    vv = W.normal(13, n * cap * hkv * d).reshape(n, cap, hkv * d)
    kstore = np.stack([W.to_kt(kl[i], cap) for i in range(n)]) if kt else kl.reshape(n, cap, hkv * d)
    sh = AttnShape(1, cap, h, hkv, d, h * d, hkv * d, h * d, True, cap if kt else None)
    out = torch.full((n, h * d), 5.0, device="cuda")
    nkv = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    ctx.attention_batch_dev(dev(torch, q), dev(torch, kstore), dev(torch, vv), sh, out, n, h * d, kstore[0].size,
                            cap * hkv * d, h * d, nkv)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, L in enumerate(lengths):
        shi = AttnShape(1, L, h, hkv, d, h * d, hkv * d, h * d, True, None)
        ref = naive.attention_f64(q[i], kl[i, :L].reshape(-1), vv[i, :L].reshape(-1), shi)
        check(got[i], ref, f"ragged item n_kv={L} ({'kt' if kt else 'row-major'})")


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("n_q", [1, 150])
def test_kt_padding_never_reaches_the_output(torch, request, mode, n_q):
    """A transposed cache's columns past n_kv (and cache rows past n_kv of V) hold NaN: the kernels
    read the padding but mask every key past n_kv by selection, so the result is the f64 closed
    form of the first n_kv keys.  (The reference asks for finite padding, src/ops.zig:477-492;
    this holds beyond that contract.)  Dense (n_q = 150, both modes, causal) and decode (n_q = 1)."""
    ctx = mode_ctx(request, mode)
    n_kv, cap, h, hkv, d = 700, 1024, 6, 2, 64
    q = W.normal(21, n_q * h * d).reshape(n_q, h * d)
    kl = W.normal(22, n_kv * hkv * d).reshape(n_kv, hkv, d)
    v = W.normal(23, n_kv * hkv * d).reshape(n_kv, hkv * d)
    kt = np.full((hkv, d, cap), np.nan, np.float32)
    kt[:, :, :n_kv] = np.transpose(kl, (1, 2, 0))
    vpad = np.full((cap, hkv * d), np.nan, np.float32)
    vpad[:n_kv] = v
    sh = AttnShape(n_q, n_kv, h, hkv, d, h * d, hkv * d, h * d, True, cap)
    out = torch.empty(n_q * h * d, device="cuda")
    ctx.attention_dev(dev(torch, q), dev(torch, kt), dev(torch, vpad), sh, out)
    torch.cuda.synchronize()
    ref = naive.attention_f64(q, kt, v, sh)
    check(out.cpu().numpy(), ref, f"NaN padding n_q={n_q} ({mode})", x3=mode == "x3" and n_q > 1)


def test_split_and_unsplit_agree(torch):
    """A context too small for split partials runs every call unsplit; results must agree."""
    import zwhisper_amd as z

    sh = AttnShape(1, 4096, 12, 2, 128, 1536, 256, 1536, True, 4096)
    q = W.normal(21, 1536)
    kl = W.normal(22, 4096 * 256).reshape(4096, 2, 128)
    kt = W.to_kt(kl, 4096)
    v = W.normal(23, 4096 * 256)
    ref = naive.attention_f64(q, kt, v, sh)
    outs = []
    for ws in (0, 1):
        with z.Context(0, workspace_bytes=ws) as c:
            out = torch.empty(1536, device="cuda")
            c.attention_dev(dev(torch, q), dev(torch, kt), dev(torch, v), sh, out)
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
            check(outs[-1], ref, f"decode, workspace {'default' if ws == 0 else 'none'}")
    sh2 = AttnShape(700, 900, 4, 4, 64, 256, 256, 256, True, None)
    q2, k2, v2 = W.normal(31, 700 * 256), W.normal(32, 900 * 256), W.normal(33, 900 * 256)
    ref2 = naive.attention_f64(q2, k2, v2, sh2)
    for ws in (0, 1):
        with z.Context(0, workspace_bytes=ws) as c:
            out = torch.empty(700 * 256, device="cuda")
            c.attention_dev(dev(torch, q2), dev(torch, k2), dev(torch, v2), sh2, out)
            torch.cuda.synchronize()
            check(out.cpu().numpy(), ref2, f"dense causal, workspace {'default' if ws == 0 else 'none'}")


@pytest.mark.parametrize("scale", [1.0, 6.0])
def test_dense_math_modes(torch, scale):
    """Both dense kernels (x3 16-bit and fp32 MFMA) against f64, on ordinary scores and on scores
    scaled up until the softmax is nearly one-hot (where the split terms carry the result);
    switching a context's mode applies to the next call, and an unknown mode is refused."""
    import zwhisper_amd as z

    sh = AttnShape(333, 777, 4, 4, 64, 256, 256, 256, False, 784)
    q = W.normal(51, 333 * 256) * scale
    kl = W.normal(52, 777 * 256).reshape(777, 4, 64) * scale
    kt = W.to_kt(kl, 784)
    v = W.normal(53, 777 * 256)
    ref = naive.attention_f64(q, kt, v, sh)
    outs = {}
    with z.Context(0) as c:
        for mode in (z.DENSE_X3, z.DENSE_FP32, z.DENSE_X3):
            c.set_dense_math(mode)
            out = torch.empty(333 * 256, device="cuda")
            c.attention_dev(dev(torch, q), dev(torch, kt), dev(torch, v), sh, out)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            # on unit-variance inputs each mode meets its own bar; with scores spread 36x wider both
            # are held to the f32 bar (measured 4.5e-5 for x3, 5.2e-5 for fp32)
            check(got, ref, f"dense mode {mode}, scores x{scale * scale:g}", x3=mode == z.DENSE_X3 and scale == 1.0)
            if mode in outs:
                assert np.array_equal(outs[mode], got), "same mode, same inputs: results differ"
            outs[mode] = got
        assert not np.array_equal(outs[z.DENSE_X3], outs[z.DENSE_FP32]), "mode switch had no effect"
        with pytest.raises(z.ZwgError):
            c.set_dense_math(7)


DENSE_SHAPES = [
    # (n_q, n_kv, heads, kv heads, d, causal, kt): every dense instantiation of both kernels
    (300, 300, 12, 2, 128, True, True),    # Qwen2-1.5B prefill, transposed K, d = 128
    (200, 333, 4, 4, 128, False, True),    # d = 128, transposed K, non-causal, ragged tiles
    (150, 260, 6, 6, 32, False, True),     # d = 32, transposed K
    (97, 97, 12, 12, 32, True, False),     # d = 32, row-major K, causal
    (129, 400, 8, 2, 64, True, False),     # d = 64, row-major K, GQA, n_kv > n_q causal
]


@pytest.mark.parametrize("mode", ["x3", "fp32"])
@pytest.mark.parametrize("shape", DENSE_SHAPES, ids=[f"q{a}k{b}h{c}g{e}d{f}{'c' if g else ''}{'kt' if h else 'rm'}"
                                                      for a, b, c, e, f, g, h in DENSE_SHAPES])
def test_dense_instantiations(torch, shape, mode):
    """Each (d, K layout) instantiation of both dense kernels against f64, with partial last tiles
    on both axes and key splits where the planner chooses them."""
    import zwhisper_amd as z

    n_q, n_kv, h, hkv, d, causal, kt = shape
    ktw = (n_kv + 7) // 8 * 8 if kt else None
    sh = AttnShape(n_q, n_kv, h, hkv, d, h * d, hkv * d, h * d, causal, ktw)
    q = W.normal(61, n_q * h * d)
    kl = W.normal(62, n_kv * hkv * d).reshape(n_kv, hkv, d)
    v = W.normal(63, n_kv * hkv * d)
    k = W.to_kt(kl, ktw) if kt else kl.reshape(-1)
    ref = naive.attention_f64(q, k, v, sh)
    with z.Context(0, dense_math=z.DENSE_X3 if mode == "x3" else z.DENSE_FP32) as c:
        out = torch.empty(n_q * h * d, device="cuda")
        c.attention_dev(dev(torch, q), dev(torch, k), dev(torch, v), sh, out)
        torch.cuda.synchronize()
        check(out.cpu().numpy(), ref, f"dense {mode} {shape}", x3=mode == "x3")


def test_x3_key_range(torch):
    """The x3 dense mode's documented range condition: a key of magnitude >= 65504 (beyond f16)
    gives NaN in exactly the rows that see it -- never a wrong finite value -- while rows the
    causal mask hides it from are unaffected; the fp32 mode handles it exactly."""
    import zwhisper_amd as z

    n_q = n_kv = 96
    h, d = 2, 64
    sh = AttnShape(n_q, n_kv, h, h, d, h * d, h * d, h * d, True, None)
    q = W.normal(71, n_q * h * d) * 0.01  # small q: the scores stay moderate even with the big key
    k = W.normal(72, n_kv * h * d).reshape(n_kv, h * d)
    v = W.normal(73, n_kv * h * d)
    big = 50                       # key row 50, head 0, one dim
    k[big, 3] = 1.0e5
    k = k.reshape(-1)
    ref = naive.attention_f64(q, k, v, sh).reshape(n_q, h * d)
    outs = {}
    for mode in (z.DENSE_X3, z.DENSE_FP32):
        with z.Context(0, dense_math=mode) as c:
            out = torch.empty(n_q * h * d, device="cuda")
            c.attention_dev(dev(torch, q), dev(torch, k), dev(torch, v), sh, out)
            torch.cuda.synchronize()
            outs[mode] = out.cpu().numpy().reshape(n_q, h * d)
    x3, f32 = outs[z.DENSE_X3], outs[z.DENSE_FP32]
    check(f32, ref, "fp32 mode with a key of 1e5", x3=False)
    # causal: query i sees keys <= i, so rows < 50 never see the big key
    check(x3[:big, :d], ref[:big, :d], "x3 rows before the big key, head 0")
    check(x3[:, d:], ref[:, d:], "x3 head 1 (no big key)")
    assert np.all(np.isnan(x3[big:, :d])), "x3 rows that see the big key must be NaN"


def test_deterministic_and_on_a_side_stream(torch, ctx):
    sh = AttnShape(300, 1000, 6, 6, 64, 384, 384, 384, False, None)
    q, k, v = (dev(torch, W.normal(s, n)) for s, n in ((41, 300 * 384), (42, 1000 * 384), (43, 1000 * 384)))
    a = torch.empty(300 * 384, device="cuda")
    b = torch.empty(300 * 384, device="cuda")
    ctx.attention_dev(q, k, v, sh, a)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ctx.attention_dev(q, k, v, sh, b)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_zero_queries_is_a_no_op(torch, ctx):
    out = torch.full((64,), 3.0, device="cuda")
    x = torch.zeros(64, device="cuda")
    ctx.attention_dev(x, x, x, AttnShape(0, 4, 1, 1, 64, 64, 64, 64, False), out)
    torch.cuda.synchronize()
    assert torch.all(out == 3.0)


def test_host_dropin_matches_device_path(torch, ctx):
    """ops.attention's drop-in (host pointers, synchronous) on the encoder's own call form."""
    import zwhisper_amd as z

    n, ns, h = 1500, 384, 6
    q, k, v = W.normal(51, n * ns), W.normal(52, n * ns), W.normal(53, n * ns)
    out = np.zeros(n * ns, np.float32)
    z.attention(None, q, k, v, n, n, ns, h, False, None, out)
    sh = AttnShape(n, n, h, h, ns // h, ns, ns, ns, False)
    check(out, naive.attention_f64(q, k, v, sh), "ops.attention drop-in, 1500 x 384")


def test_x3_dropin_recomputes_out_of_range_keys(ctx):
    """zwg_attention_ex keeps the reference's contract for any finite input: a key beyond f16
    range (NaN rows on the x3 kernel) makes the drop-in compute the call again on the fp32
    kernel, so every row is finite and within the f32 bar of f64."""
    n_q = n_kv = 96
    h, d = 2, 64
    sh = AttnShape(n_q, n_kv, h, h, d, h * d, h * d, h * d, True, None)
    q = W.normal(81, n_q * h * d) * 0.01
    k = W.normal(82, n_kv * h * d).reshape(n_kv, h * d)
    k[40, 5] = -2.0e5
    k = k.reshape(-1)
    v = W.normal(83, n_kv * h * d)
    out = np.zeros(n_q * h * d, np.float32)
    ctx.attention_ex_host(q, k, v, sh, out)
    check(out, naive.attention_f64(q, k, v, sh), "drop-in with a key of -2e5", x3=False)


def test_two_unordered_streams_share_the_workspace(torch, ctx):
    """Two split calls of one context on two streams that do not wait for each other: the
    context orders the second stream after the first when it switches (both write their split
    partials to the same workspace), so both results are right."""
    sh = AttnShape(1, 3000, 12, 2, 128, 1536, 256, 1536, True, 3000)
    import zwhisper_amd as z

    assert z.plan(sh).max_chunks > 1, "the case must split its keys"
    inputs, refs = [], []
    for seed in (91, 95):
        q = W.normal(seed, 1536)
        kl = W.normal(seed + 1, 3000 * 256).reshape(3000, 2, 128)
        kt = W.to_kt(kl, 3000)
        v = W.normal(seed + 2, 3000 * 256)
        inputs.append((dev(torch, q), dev(torch, kt), dev(torch, v), torch.empty(1536, device="cuda")))
        refs.append(naive.attention_f64(q, kt, v, sh))
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(sa):
            q, k, v, o = inputs[0]
            ctx.attention_dev(q, k, v, sh, o)
        with torch.cuda.stream(sb):
            q, k, v, o = inputs[1]
            ctx.attention_dev(q, k, v, sh, o)
        torch.cuda.synchronize()
        for (_, _, _, o), ref, name in zip(inputs, refs, ("stream a", "stream b")):
            check(o.cpu().numpy(), ref, f"decode on {name}")


def test_children_outlive_their_closed_context(torch):
    """zwg_close frees the device memory of caches and int8 weights made from the context and not
    destroyed yet; the orphaned objects then refuse to be used and can still be destroyed."""
    import zwhisper_amd as z

    c = z.Context(0)
    kv = z.KVCache(c, 1, 1, 64, 2, 64)
    rng = np.random.default_rng(5)
    w = z.Q8(rng.integers(-127, 128, (64, 64), dtype=np.int8), np.ones((64, 2), np.float32), 64, 64).resident(c)
    c._children.clear()  # bypass the Python-side close of the children: the C ABI's own rule
    c.close()
    x = torch.zeros(64, device="cuda")
    out = torch.empty(64, device="cuda")
    with z.Context(0) as c2:
        with pytest.raises(z.ZwgError):
            c2.linear_q8w_dev(x, 1, w, None, out)
    with pytest.raises(z.ZwgError):
        kv.read(0, 0)
    kv.close()
    w.close()


@pytest.mark.parametrize("n_items,kt", [(300, True), (300, False), (256, True)])
def test_decode_many_ragged_items(torch, ctx, n_items, kt):
    """Per-item key counts over more items than the decode kernels map onto the list of non-empty
    chunks (256): those calls keep the plain (item, chunk, KV head) grid.  Both grids, both key
    layouts, every item against f64."""
    cap, h, hkv, d = 512, 4, 2, 64
    rng = np.random.default_rng(n_items)
    lengths = rng.integers(0, cap + 1, n_items).astype(np.int32)
    lengths[:3] = [0, 1, cap]
    q = W.normal(101, n_items * h * d).reshape(n_items, h * d)
    kl = W.normal(102, n_items * cap * hkv * d).reshape(n_items, cap, hkv, d)
    v = W.normal(103, n_items * cap * hkv * d).reshape(n_items, cap, hkv * d)
    kstore = np.stack([W.to_kt(kl[i], cap) for i in range(n_items)]) if kt else kl.reshape(n_items, cap, hkv * d)
    sh = AttnShape(1, cap, h, hkv, d, h * d, hkv * d, h * d, False, cap if kt else None)
    out = torch.full((n_items, h * d), 9.0, device="cuda")
    ctx.attention_batch_dev(dev(torch, q), dev(torch, kstore), dev(torch, v), sh, out, n_items, h * d,
                            kstore[0].size, cap * hkv * d, h * d, torch.from_numpy(lengths).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i in range(n_items):
        L = int(lengths[i])
        if L == 0:
            assert np.all(got[i] == 0.0), f"item {i} with no keys must give zeros"
            continue
        shi = AttnShape(1, L, h, hkv, d, h * d, hkv * d, h * d, False, None)
        ref = naive.attention_f64(q[i], kl[i, :L].reshape(-1), v[i, :L].reshape(-1), shi)
        check(got[i], ref, f"{n_items} items, item {i} n_kv={L} ({'kt' if kt else 'row-major'})")


def test_x3_value_range(torch, ctx):
    """The x3 dense mode's value-range condition: a value of magnitude >= 65504 (beyond f16) gives
    NaN in its own output column (its head and dimension) of the rows that load its 32-key tile --
    never a wrong finite result -- while the fp32 mode and the host drop-in (which recomputes such
    a call in fp32) stay within the f32 bar."""
    import zwhisper_amd as z

    n_q = n_kv = 96
    h, d = 2, 64
    sh = AttnShape(n_q, n_kv, h, h, d, h * d, h * d, h * d, True, None)
    q = W.normal(74, n_q * h * d)
    k = W.normal(75, n_kv * h * d)
    v = W.normal(76, n_kv * h * d).reshape(n_kv, h * d)
    v[70, 7] = 2.0e5  # key 70 (third 32-key tile), head 0, dimension 7
    v = v.reshape(-1)
    ref = naive.attention_f64(q, k, v, sh).reshape(n_q, h * d)
    with z.Context(0, dense_math=z.DENSE_FP32) as c:
        out = torch.empty(n_q * h * d, device="cuda")
        c.attention_dev(dev(torch, q), dev(torch, k), dev(torch, v), sh, out)
        torch.cuda.synchronize()
        check(out.cpu().numpy().reshape(n_q, h * d), ref, "fp32 mode with a value of 2e5", x3=False, v_scale=2.0e5)
    out = torch.empty(n_q * h * d, device="cuda")
    ctx.attention_dev(dev(torch, q), dev(torch, k), dev(torch, v), sh, out)
    torch.cuda.synchronize()
    x3 = out.cpu().numpy().reshape(n_q, h * d)
    # causal: the waves of queries < 64 never load the tile of keys 64..95, so column 7 is exact
    # there; every other column of every row, and all of head 1, never meets the big value
    other = np.ones(h * d, bool)
    other[7] = False
    check(x3[:, other], ref[:, other], "x3 columns without the big value")
    check(x3[:64, 7], ref[:64, 7], "x3 column 7, rows before the big value's tile")
    # rows 70.. see key 70: hi term +inf, lo term -inf, so NaN; rows 64..69 mask it (p = 0, and
    # 0 * inf is NaN in IEEE arithmetic): NaN or, were the product flushed, the exact value
    assert np.all(np.isnan(x3[70:, 7])), "x3 column 7 of the rows that see the big value must be NaN"
    masked = x3[64:70, 7]
    fin = np.isfinite(masked)
    print(f"x3 column 7, rows 64..69 (big value masked): {int(np.sum(~fin))} of 6 NaN", flush=True)
    if fin.any():
        check(masked[fin], ref[64:70, 7][fin], "x3 column 7, finite rows 64..69")
    host = np.zeros(n_q * h * d, np.float32)
    ctx.attention_ex_host(q, k, v, sh, host)
    check(host, ref, "drop-in with a value of 2e5", x3=False, v_scale=2.0e5)
