"""GPU parity of the linear layer over int8 block weights (zwg_linear_q8 / zwg_linear_q8_dev)
against the f64 closed form over the dequantized weights and the oracle's ops.linear with a Q8
(src/ops.zig:283-306, gemm.ntBlockQ / micro4x4Q / dotQ, src/gemm.zig:274-351).

Bar: max abs error <= 2e-5 * sqrt(k) on outputs of unit scale (x ~ N(0, 1), weights quantized
from N(0, 1/k)), the size of the reference's own f32 accumulation error, and never worse than the
oracle by more than that.  Known answers: a one-hot int8 row with scale 1 gives exactly the
two-term split's value of x, f32(hi + lo); scales that are powers of two scale it exactly.
Shapes: the Whisper small.en decoder step over 32 windows and the Qwen2.5 decode step over 64
sequences (the weight-streaming kernel, m <= 64, with and without the k split), their logits,
and prefill-sized calls (the tiled kernel).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


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


def inputs(seed, m, k, n, bias=True):
    import zwhisper_amd as z

    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float32) if bias else None
    return x, z.Q8.quantize(w, n, k), b


def run_dev(torch, ctx, x, w, b, m, k, n):
    out = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_q8_dev(torch.from_numpy(x).cuda(), m, k, w.to_device(),
                      None if b is None else torch.from_numpy(b).cuda(), n, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def ref64(x, w, b):
    deq = oracle.q8_dequantize(w.q, w.scales).astype(np.float64)
    r = x.astype(np.float64) @ deq.T
    return r if b is None else r + b.astype(np.float64)[None, :]


CASES = [
    # Whisper small.en decoder step, 32 windows (src/decoder.zig:181-205): q/k/v/o, MLP up, down
    (32, 768, 768), (32, 768, 3072), (32, 3072, 768),
    # Qwen2.5-1.5B decode step, 64 sequences (src/llm.zig:179-216): q/o, k/v, gate/up, down
    (64, 1536, 1536), (64, 1536, 256), (64, 1536, 8960), (64, 8960, 1536),
    # Qwen2.5-0.5B single-sequence decode and small batches
    (1, 896, 896), (1, 896, 4864), (2, 4864, 896), (17, 896, 128), (33, 896, 896),
    # prefill-sized: Qwen2.5-0.5B 256-row batch (src/llm.zig:258-266), a Whisper window's cross K/V
    # (src/decoder.zig:151-159), tails in m, n and k
    (256, 896, 896), (256, 896, 4864), (1500, 768, 768), (65, 96, 130), (129, 544, 257), (100, 32, 3),
]


@pytest.mark.parametrize("m,k,n", CASES)
def test_linear_q8_matches_reference(torch, ctx, m, k, n):
    x, w, b = inputs(m * 7 + n + k, m, k, n)
    got = run_dev(torch, ctx, x, w, b, m, k, n)
    ref = ref64(x, w, b)
    err = float(np.abs(got - ref).max())
    bar = 2e-5 * np.sqrt(k)
    print(f"linear q8 {m}x{k}x{n}: max abs {err:.2e} (bar {bar:.1e})", flush=True)
    assert np.all(np.isfinite(got)) and err <= bar
    if m * n * k <= 60_000_000:
        with oracle.Oracle(4) as o:
            ora = o.linear_q8(x, m, k, w.q, w.scales, b, n).reshape(m, n)
        assert float(np.abs(got - ora).max()) <= err + bar


@pytest.mark.parametrize("m,k,n", [(64, 1536, 151936), (32, 768, 51864)])
def test_logits(torch, ctx, m, k, n):
    """The output projection over the whole vocabulary (Qwen2.5 tied embeddings, src/llm.zig:214-216;
    Whisper small.en, src/decoder.zig:203-205), checked in f64 on the device."""
    rng = np.random.default_rng(n)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    q = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=torch.Generator().manual_seed(n)).cuda()
    sc = (torch.rand(n, k // 32, generator=torch.Generator().manual_seed(n + 1)) * (2.0 / 127 / np.sqrt(k))).cuda()
    import zwhisper_amd as z

    out = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_q8_dev(x, m, k, z.Q8(q, sc, n, k), None, n, out)
    deq = (q.double().view(n, k // 32, 32) * sc.double().view(n, k // 32, 1)).view(n, k)
    ref = x.double() @ deq.T
    err = float((out.double() - ref).abs().max())
    bar = 2e-5 * np.sqrt(k)
    print(f"logits q8 {m}x{k}x{n}: max abs {err:.2e} (bar {bar:.1e})", flush=True)
    assert bool(torch.isfinite(out).all()) and err <= bar


def split_value(x):
    """f32(hi + lo) with hi = f16(x), lo = f16(x - hi): what one weight of 1 passes through."""
    hi = x.astype(np.float16).astype(np.float32)
    lo = (x - hi).astype(np.float16).astype(np.float32)
    return (hi + lo).astype(np.float32)


@pytest.mark.parametrize("m", [5, 40, 300])
def test_one_hot_and_power_of_two_scales(torch, ctx, m):
    """One nonzero int8 per weight row: out = q * scale * split(x), exact for q*scale a power of two."""
    import zwhisper_amd as z

    k, n = 96, 6
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    q = np.zeros((n, k), np.int8)
    sc = np.zeros((n, k // 32), np.float32)
    picks = [(0, 0, 1, 1.0), (1, 31, 1, 0.5), (2, 32, -1, 4.0), (3, 95, 2, 0.25), (4, 64, 64, 2.0 ** -6),
             (5, 50, -128 + 1, 1.0)]
    for o, p, v, s in picks:
        q[o, p] = v
        sc[o, p // 32] = s
    got = run_dev(torch, ctx, x, z.Q8(q, sc, n, k), None, m, k, n)
    for o, p, v, s in picks[:5]:
        assert np.array_equal(got[:, o], (split_value(x[:, p]) * np.float32(v * s)).astype(np.float32)), o
    ref = x[:, 50].astype(np.float64) * -127.0
    assert np.max(np.abs(got[:, 5] - ref)) <= 127 * 2.0 ** -21 * np.max(np.abs(x[:, 50]))


def test_split_and_unsplit_agree(torch, ctx):
    """The k split (few weight rows, long k) and the tiled kernel give the same sums within the bar."""
    m, k, n = 64, 8960, 256
    x, w, b = inputs(5, m, k, n)
    small = run_dev(torch, ctx, x, w, b, m, k, n)          # m <= 64: streaming kernel, split over k
    big = run_dev(torch, ctx, np.concatenate([x, x[:1]]), w, b, m + 1, k, n)[:m]  # tiled kernel
    ref = ref64(x, w, b)
    bar = 2e-5 * np.sqrt(k)
    assert float(np.abs(small - ref).max()) <= bar and float(np.abs(big - ref).max()) <= bar


def test_deterministic(torch, ctx):
    m, k, n = 64, 1536, 1536
    x, w, b = inputs(8, m, k, n)
    a = run_dev(torch, ctx, x, w, b, m, k, n)
    c = run_dev(torch, ctx, x, w, b, m, k, n)
    assert np.array_equal(a, c)


def test_host_dropin(torch, ctx):
    """zwhisper_amd.linear with a Q8: ops.linear's call form on host arrays."""
    import zwhisper_amd as z

    for m, k, n in ((3, 128, 96), (200, 256, 72)):
        x, w, b = inputs(9 + m, m, k, n)
        out = np.zeros(m * n, np.float32)
        z.linear(None, x.reshape(-1), m, k, w, b, n, out)
        assert float(np.abs(out.reshape(m, n) - ref64(x, w, b)).max()) <= 2e-5 * np.sqrt(k)


def test_linear_q8_errors(torch, ctx):
    import zwhisper_amd as z

    t = torch.zeros(4096, device="cuda")
    w = z.Q8(torch.zeros((4, 48 * 2), dtype=torch.int8, device="cuda"), torch.zeros((4, 3), device="cuda"), 4, 96)
    w.k = 48  # a k that is not a multiple of 32 must be refused by the library itself
    with pytest.raises(z.ZwgError, match="multiple of 32"):
        ctx.linear_q8_dev(t, 2, 48, w, None, 4, t)
    w2 = z.Q8(torch.zeros((4, 64), dtype=torch.int8, device="cuda"), torch.zeros((4, 2), device="cuda"), 4, 64)
    with pytest.raises(z.ZwgError, match="asks for"):
        ctx.linear_q8_dev(t, 2, 64, w2, None, 5, t)


@pytest.mark.parametrize("m,k,n", CASES)
def test_resident_packed_matches_raw(torch, ctx, m, k, n):
    """Weights uploaded once in the packed device layout (zwg_q8w) give the raw-layout call's
    results bit for bit at these shapes, where both paths split k into the same pieces: the same
    arithmetic, only the weight loads differ.  (Where the splits differ -- at m <= 32 the packed
    kernel's workgroups cover half as many weight rows -- the two agree to rounding;
    test_gpu_linear_fuzz.py checks both against f64 over random shapes.)  Calls of 65..256 rows
    stream the packed weights in 64-row blocks where the raw path tiles: there the two agree to
    rounding and each is checked against f64."""
    x, w, b = inputs(m * 11 + n + k, m, k, n)
    raw = run_dev(torch, ctx, x, w, b, m, k, n)
    xd = torch.from_numpy(x).cuda()
    bd = torch.from_numpy(b).cuda()
    for src in (w, w.to_device()):  # packed from host arrays and from device tensors
        with src.resident(ctx) as rw:
            out = torch.full((m, n), float("nan"), device="cuda")
            ctx.linear_q8w_dev(xd, m, rw, bd, out)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            if 64 < m <= 256:
                ref = ref64(x, w, b)
                assert np.all(np.isfinite(got))
                assert float(np.abs(got - ref).max()) <= 2e-5 * np.sqrt(k)
                assert float(np.abs(got - raw).max()) <= 2e-5 * np.sqrt(k)
            else:
                assert np.array_equal(got, raw)


def test_resident_logits(torch, ctx):
    """The Qwen2.5-1.5B vocabulary projection from resident packed weights, against f64."""
    import zwhisper_amd as z

    m, k, n = 64, 1536, 151936
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
    q = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=torch.Generator().manual_seed(4)).cuda()
    sc = (torch.rand(n, k // 32, generator=torch.Generator().manual_seed(5)) * (2.0 / 127 / np.sqrt(k))).cuda()
    with z.Q8(q, sc, n, k).resident(ctx) as rw:
        out = torch.full((m, n), float("nan"), device="cuda")
        ctx.linear_q8w_dev(x, m, rw, None, out)
        torch.cuda.synchronize()
    deq = (q.double().view(n, k // 32, 32) * sc.double().view(n, k // 32, 1)).view(n, k)
    err = float((out.double() - x.double() @ deq.T).abs().max())
    assert bool(torch.isfinite(out).all()) and err <= 2e-5 * np.sqrt(k)


GROUPS = [
    # Qwen2.5-1.5B q/k/v (src/llm.zig:179-190): biased, biased, biased; Whisper q/k/v: k unbiased
    (1536, [(1536, True), (256, True), (256, True)]),
    (768, [(768, True), (768, False), (768, True)]),
    # Qwen2.5-1.5B MLP gate and up (src/llm.zig:203-205)
    (1536, [(8960, False), (8960, False)]),
    # four sets, none a multiple of 128 rows, mixed biases
    (544, [(130, True), (33, False), (257, True), (96, False)]),
]


@pytest.mark.parametrize("m", [64, 33, 17, 1, 100])
@pytest.mark.parametrize("gi", range(len(GROUPS)))
def test_resident_group(torch, ctx, m, gi):
    """zwg_linear_q8w_group_dev: each output against its single call (to f32 rounding: the group's
    k split can differ from a single call's), against f64, and the same call twice bit for bit;
    m = 100 takes two 64-row blocks of the stream kernel in one launch."""
    import contextlib

    k, sets = GROUPS[gi]
    print(f"group {gi} m={m} k={k} sets={sets}", flush=True)
    rng = np.random.default_rng(100 + gi * 7 + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    qs, bs = [], []
    for j, (n, hb) in enumerate(sets):
        _, w, b = inputs(1000 + 13 * gi + j, 1, k, n, bias=hb)
        qs.append(w)
        bs.append(None if b is None else torch.from_numpy(b).cuda())
    with contextlib.ExitStack() as stack:
        rs = [stack.enter_context(w.resident(ctx)) for w in qs]
        outs = [torch.full((m, w.n), float("nan"), device="cuda") for w in rs]
        ctx.linear_q8w_group_dev(xd, m, rs, bs, outs)
        again = [torch.full((m, w.n), float("nan"), device="cuda") for w in rs]
        ctx.linear_q8w_group_dev(xd, m, rs, bs, again)
        singles = []
        for r, b in zip(rs, bs):
            o = torch.full((m, r.n), float("nan"), device="cuda")
            ctx.linear_q8w_dev(xd, m, r, b, o)
            singles.append(o)
        torch.cuda.synchronize()
        for j, (w, b) in enumerate(zip(qs, bs)):
            got, single = outs[j].cpu().numpy(), singles[j].cpu().numpy()
            assert np.all(np.isfinite(got)), j
            assert np.array_equal(got, again[j].cpu().numpy()), f"set {j}: not deterministic"
            ref = ref64(x, w, None if b is None else b.cpu().numpy())
            assert float(np.abs(got - ref).max()) <= 2e-5 * np.sqrt(k), f"set {j}: against f64"
            assert float(np.abs(got - single).max()) <= 1e-6 * max(1.0, float(np.abs(single).max())), \
                f"set {j}: against the single call"


def test_resident_group_errors(torch, ctx):
    import zwhisper_amd as z

    _, w1, _ = inputs(1, 1, 256, 64, bias=False)
    _, w2, _ = inputs(2, 1, 512, 64, bias=False)
    x = torch.zeros(4 * 512, device="cuda")
    out = [torch.zeros(4 * 64, device="cuda"), torch.zeros(4 * 64, device="cuda")]
    with w1.resident(ctx) as r1, w2.resident(ctx) as r2:
        with pytest.raises(z.ZwgError, match="share k"):
            ctx.linear_q8w_group_dev(x, 4, [r1, r2], None, out)
        with pytest.raises(z.ZwgError):
            ctx.linear_q8w_group_dev(x, 4, [r1] * 5, None, out * 3)


def test_split_calls_in_graph_replays(torch, ctx):
    """A Whisper small.en decode step's k-split calls (q/k/v grouped, split 3; MLP up, split 3; MLP
    down, split 12), captured in a HIP graph: every replay, with eager calls of other inputs between
    replays, gives the eager results bit for bit."""
    import contextlib

    m = 32
    rng = np.random.default_rng(21)
    shapes = [(768, 768, True), (768, 768, False), (768, 768, True), (768, 3072, True), (3072, 768, True)]
    ws, bs = [], []
    for j, (k, n, hb) in enumerate(shapes):
        _, w, b = inputs(400 + j, 1, k, n, bias=hb)
        ws.append(w)
        bs.append(None if b is None else torch.from_numpy(b).cuda())
    x768 = torch.from_numpy(rng.standard_normal((m, 768)).astype(np.float32)).cuda()
    x3072 = torch.from_numpy(rng.standard_normal((m, 3072)).astype(np.float32)).cuda()
    other768, other3072 = x768.flip(0).contiguous(), x3072.flip(0).contiguous()
    with contextlib.ExitStack() as stack:
        rs = [stack.enter_context(w.resident(ctx)) for w in ws]

        def step(a768, a3072):
            outs = [torch.empty((m, r.n), device="cuda") for r in rs]
            ctx.linear_q8w_group_dev(a768, m, rs[:3], bs[:3], outs[:3])
            ctx.linear_q8w_dev(a768, m, rs[3], bs[3], outs[3])
            ctx.linear_q8w_dev(a3072, m, rs[4], bs[4], outs[4])
            return outs

        eager = [o.cpu().numpy() for o in step(x768, x3072)]
        for j, (w, b) in enumerate(zip(ws, bs)):
            xin = x768 if shapes[j][0] == 768 else x3072
            ref = ref64(xin.cpu().numpy(), w, None if b is None else b.cpu().numpy())
            assert float(np.abs(eager[j] - ref).max()) <= 2e-5 * np.sqrt(shapes[j][0]), f"call {j}: against f64"
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = step(x768, x3072)
        for rep in range(3):
            for o in captured:
                o.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            for j in range(len(shapes)):
                assert np.array_equal(captured[j].cpu().numpy(), eager[j]), f"replay {rep}, call {j}"
            step(other768, other3072)  # eager calls between replays
            torch.cuda.synchronize()


# Unsplit calls of 128-255 workgroups (resident weights): each workgroup's waves form two groups,
# each over half of the stages of 128 k, summed through LDS.  Shapes: the Qwen2.5-1.5B MLP gate
# (m = 64 and 33, two m-tiles), a 32-row call (one m-tile, x split in the stream kernel), and k
# whose stage count is odd or leaves the second group one stage (k = 416: 4 stages, the last
# partial; k = 384: 3 stages; k = 288: 3 stages, the last a quarter).
TWO_GROUP_CASES = [(64, 1536, 17920), (33, 416, 16400), (32, 384, 9000), (17, 8960, 9000), (1, 288, 12000)]


@pytest.mark.parametrize("m,k,n", TWO_GROUP_CASES)
def test_two_stage_groups(torch, ctx, m, k, n):
    x, w, b = inputs(m * 5 + n + k, m, k, n)
    xd, bd = torch.from_numpy(x).cuda(), torch.from_numpy(b).cuda()
    ref = ref64(x, w, b)
    with w.resident(ctx) as rw:
        outs = []
        for _ in range(2):
            out = torch.full((m, n), float("nan"), device="cuda")
            ctx.linear_q8w_dev(xd, m, rw, bd, out)
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
    err = float(np.abs(outs[0] - ref).max())
    bar = 2e-5 * np.sqrt(k)
    print(f"two stage groups q8 {m}x{k}x{n}: max abs {err:.2e} (bar {bar:.1e})", flush=True)
    assert np.all(np.isfinite(outs[0])) and err <= bar
    assert np.array_equal(outs[0], outs[1])
