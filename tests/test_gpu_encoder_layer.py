"""GPU parity of the encoder-layer pieces and of a whole Whisper encoder layer (include/zw_gpu.h:
zwg_layer_norm_dev, zwg_gelu_dev, zwg_add_dev, the linear epilogues, zwg_encoder_layer_dev)
against the oracle (oracle/attn_oracle.c: ora_layer_norm, ora_gelu, ora_linear_f16,
ora_attention; Oracle.encoder_layer composes src/encoder.zig:164-175) and f64 closed forms.

Bars: layer norm and GELU within 2e-6 relative of the oracle (both are f32 restatements of the
same formulas; only sum order and the exp routine differ); the epilogues bit-exact against the
plain GEMM followed by the standalone op; a whole layer within 2e-4 max abs of the oracle's
layer on unit-scale activations (the attention bar of this build).
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


@pytest.fixture(scope="module")
def ora():
    o = oracle.Oracle(4)
    yield o
    o.close()


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("m,n,eps", [(1500, 384, 1e-5), (3000, 512, 1e-5), (33, 768, 1e-12), (5, 1280, 1e-5),
                                     (3, 4, 1e-5), (4, 2052, 1e-5), (2, 6000, 1e-5)])
def test_layer_norm(torch, ctx, ora, m, n, eps):
    rng = np.random.default_rng(m + n)
    x = (rng.standard_normal((m, n)) * rng.uniform(0.1, 20, (m, 1)) + rng.uniform(-5, 5, (m, 1))).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    out = torch.full((m, n), float("nan"), device="cuda")
    ctx.layer_norm_dev(dev(torch, x), m, n, dev(torch, w), dev(torch, b), eps, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = ora.layer_norm(x, m, n, w, b, eps)
    assert np.max(np.abs(got - ref)) <= 2e-6 * max(1.0, float(np.max(np.abs(ref))))


def test_layer_norm_constant_rows_give_b(torch, ctx):
    m, n = 8, 512
    b = np.linspace(-1, 1, n).astype(np.float32)
    out = torch.empty((m, n), device="cuda")
    ctx.layer_norm_dev(torch.full((m, n), 3.5, device="cuda"), m, n, dev(torch, np.ones(n, np.float32)),
                       dev(torch, b), 1e-5, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), np.tile(b, (m, 1)))


@pytest.mark.parametrize("size", [4, 100, 1500 * 1536, 4096 + 4])
def test_gelu(torch, ctx, ora, size):
    x = np.random.default_rng(size).standard_normal(size).astype(np.float32) * 3
    x[: min(4, size)] = [0.0, 30.0, -30.0, 1.0][: min(4, size)]
    t = dev(torch, x)
    ctx.gelu_dev(t)
    torch.cuda.synchronize()
    got = t.cpu().numpy()
    ref = ora.gelu(x)
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) <= 2e-6
    assert got[0] == 0.0
    if size >= 4:
        assert got[1] == np.float32(30.0) and got[2] == 0.0


def test_add(torch, ctx):
    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    y = np.random.default_rng(1).standard_normal(1000).astype(np.float32)
    t = dev(torch, x)
    ctx.add_dev(t, dev(torch, y))
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), x + y)


@pytest.mark.parametrize("m,k,n", [(8257, 512, 512), (8200, 512, 2048), (1500, 384, 1536), (300, 512, 512),
                                   (7, 64, 40), (200, 2048, 512)])
def test_linear_epilogues_exact(torch, ctx, m, k, n):
    """GELU and ADD epilogues equal the plain GEMM followed by zwg_gelu_dev / zwg_add_dev bit for bit,
    and the output stride writes into a wider buffer without touching the other columns.  The first
    two shapes run the 64 x 256 and 128 x 256 tiles with a last row block cut short (the ADD
    epilogue's residual loads go through a descriptor ending at the tile's last element); the last
    two split k, so the split sum's epilogue and stride are the ones checked."""
    from zwhisper_amd import _lib

    rng = np.random.default_rng(m)
    x = dev(torch, rng.standard_normal((m, k)).astype(np.float32))
    w = dev(torch, (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16))
    b = dev(torch, rng.standard_normal(n).astype(np.float32))
    plain = torch.empty((m, n), device="cuda")
    ctx.linear_epi_dev(x, m, k, w, b, n, plain, _lib.EPI_NONE)
    g = torch.empty((m, n), device="cuda")
    ctx.linear_epi_dev(x, m, k, w, b, n, g, _lib.EPI_GELU)
    base = dev(torch, rng.standard_normal((m, n)).astype(np.float32))
    acc = base.clone()
    ctx.linear_epi_dev(x, m, k, w, b, n, acc, _lib.EPI_ADD)
    wide = torch.full((m, 3 * n), 7.0, device="cuda")
    ctx.linear_epi_dev(x, m, k, w, b, n, wide.view(-1)[n:], _lib.EPI_NONE, out_stride=3 * n)
    wide_a = torch.full((m, 3 * n), 7.0, device="cuda")
    wide_a[:, n:2 * n] = base
    ctx.linear_epi_dev(x, m, k, w, b, n, wide_a.view(-1)[n:], _lib.EPI_ADD, out_stride=3 * n)
    ref_g = plain.clone()
    ctx.gelu_dev(ref_g)
    ref_a = base.clone()
    ctx.add_dev(ref_a, plain)
    torch.cuda.synchronize()
    assert torch.equal(g, ref_g) and torch.equal(acc, ref_a)
    assert torch.equal(wide[:, n:2 * n], plain) and torch.equal(wide_a[:, n:2 * n], ref_a)
    for t in (wide, wide_a):
        assert bool((t[:, :n] == 7.0).all()) and bool((t[:, 2 * n:] == 7.0).all())


@pytest.mark.parametrize("m,k,n", [(32, 768, 3072), (64, 1536, 256), (64, 8960, 1536), (300, 768, 768),
                                   (256, 4864, 896)])
def test_q8_epilogues_exact(torch, ctx, m, k, n):
    """The same for resident int8 weights: the token-step kernel, its k-split sum, and the tiled kernel
    with and without its own k split."""
    import zwhisper_amd as z
    from zwhisper_amd import _lib

    rng = np.random.default_rng(n)
    x = dev(torch, rng.standard_normal((m, k)).astype(np.float32))
    w = z.Q8.quantize((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32), n, k)
    b = dev(torch, rng.standard_normal(n).astype(np.float32))
    with w.resident(ctx) as rw:
        plain = torch.empty((m, n), device="cuda")
        ctx.linear_q8w_epi_dev(x, m, rw, b, plain, _lib.EPI_NONE)
        g = torch.empty((m, n), device="cuda")
        ctx.linear_q8w_epi_dev(x, m, rw, b, g, _lib.EPI_GELU)
        base = dev(torch, rng.standard_normal((m, n)).astype(np.float32))
        acc = base.clone()
        ctx.linear_q8w_epi_dev(x, m, rw, b, acc, _lib.EPI_ADD)
        ref_g = plain.clone()
        ctx.gelu_dev(ref_g)
        ref_a = base.clone()
        ctx.add_dev(ref_a, plain)
        torch.cuda.synchronize()
    assert torch.equal(g, ref_g) and torch.equal(acc, ref_a)


def layer_weights(rng, ns):
    def f16(n, k):
        return (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16)

    def vec(n, scale=0.1):
        return (rng.standard_normal(n) * scale).astype(np.float32)

    return {"attn_ln_w": 1 + vec(ns), "attn_ln_b": vec(ns), "q_w": f16(ns, ns), "q_b": vec(ns), "k_w": f16(ns, ns),
            "v_w": f16(ns, ns), "v_b": vec(ns), "o_w": f16(ns, ns), "o_b": vec(ns), "mlp_ln_w": 1 + vec(ns),
            "mlp_ln_b": vec(ns), "mlp0_w": f16(4 * ns, ns), "mlp0_b": vec(4 * ns), "mlp1_w": f16(ns, 4 * ns),
            "mlp1_b": vec(ns)}


@pytest.mark.parametrize("n_windows,n_ctx,ns,n_head", [(1, 1500, 384, 6), (2, 1500, 512, 8), (3, 70, 64, 2)])
def test_encoder_layer(torch, ctx, ora, n_windows, n_ctx, ns, n_head):
    """tiny.en and base.en shaped layers (and the reference test's small shape) over several windows
    at once, each window against the oracle's layer."""
    import zwhisper_amd as z

    rng = np.random.default_rng(ns)
    w = layer_weights(rng, ns)
    x = rng.standard_normal((n_windows, n_ctx, ns)).astype(np.float32)
    xd = dev(torch, x)
    scratch = torch.empty(z.ops.encoder_layer_scratch(n_windows * n_ctx, ns), device="cuda")
    ctx.encoder_layer_dev(xd, n_windows, n_ctx, ns, n_head, {kk: dev(torch, v) for kk, v in w.items()}, scratch)
    torch.cuda.synchronize()
    got = xd.cpu().numpy()
    for win in range(n_windows):
        ref = ora.encoder_layer(x[win], n_ctx, ns, n_head, w)
        err = float(np.max(np.abs(got[win] - ref)))
        print(f"encoder layer {n_ctx}x{ns} window {win}: max abs {err:.2e}", flush=True)
        assert np.all(np.isfinite(got[win])) and err <= 2e-4


def composed_layer(torch, ctx, xd, n_windows, n_ctx, ns, n_head, wd):
    """The layer from the library's public calls with q | k | v as f32 rows (the path without tile
    images): layer norm, the three projections into one [rows][3 ns] buffer, batched attention
    through its strides, then the o-projection and MLP with their fused epilogues."""
    from zwhisper_amd import _lib
    from zwhisper_amd.ops import AttnShape

    rows = n_windows * n_ctx
    a = torch.empty((rows, ns), device="cuda")
    b = torch.empty((rows, 3 * ns), device="cuda")
    ctx.layer_norm_dev(xd, rows, ns, wd["attn_ln_w"], wd["attn_ln_b"], 1e-5, a)
    flat = b.view(-1)
    ctx.linear_epi_dev(a, rows, ns, wd["q_w"], wd["q_b"], ns, flat, _lib.EPI_NONE, out_stride=3 * ns)
    ctx.linear_epi_dev(a, rows, ns, wd["k_w"], None, ns, flat[ns:], _lib.EPI_NONE, out_stride=3 * ns)
    ctx.linear_epi_dev(a, rows, ns, wd["v_w"], wd["v_b"], ns, flat[2 * ns:], _lib.EPI_NONE, out_stride=3 * ns)
    sh = AttnShape(n_ctx, n_ctx, n_head, n_head, ns // n_head, 3 * ns, 3 * ns, ns, False)
    ctx.attention_batch_dev(flat, flat[ns:], flat[2 * ns:], sh, a, n_windows, n_ctx * 3 * ns, n_ctx * 3 * ns,
                            n_ctx * 3 * ns, n_ctx * ns)
    ctx.linear_epi_dev(a, rows, ns, wd["o_w"], wd["o_b"], ns, xd, _lib.EPI_ADD)
    ctx.layer_norm_dev(xd, rows, ns, wd["mlp_ln_w"], wd["mlp_ln_b"], 1e-5, a)
    h = torch.empty((rows, 4 * ns), device="cuda")
    ctx.linear_epi_dev(a, rows, ns, wd["mlp0_w"], wd["mlp0_b"], 4 * ns, h, _lib.EPI_GELU)
    ctx.linear_epi_dev(h, rows, 4 * ns, wd["mlp1_w"], wd["mlp1_b"], ns, xd, _lib.EPI_ADD)


# (windows, frames, n_state, heads): base.en and tiny.en windows (1500 frames: the last 32-key tile
# holds 28 keys), head dim 128 with a last tile of 4 keys, whole tiles only, and 70 frames (not a
# multiple of 4: no images, the f32 path)
IMAGE_SHAPES = [(2, 1500, 512, 8), (1, 1500, 384, 6), (2, 68, 256, 2), (3, 64, 128, 2), (2, 70, 128, 2)]


@pytest.mark.parametrize("n_windows,n_ctx,ns,n_head", IMAGE_SHAPES)
def test_encoder_layer_images_match_f32_rows(torch, ctx, n_windows, n_ctx, ns, n_head):
    """In the x3 mode the layer's K and V projections write tile images that attention copies into
    LDS as they are; the f16 terms are the ones attention would form from f32 rows, so the layer
    equals the composed f32-row layer bit for bit (the scratch is filled with NaN first, so an
    unwritten padding key would show)."""
    import zwhisper_amd as z

    rng = np.random.default_rng(ns + n_ctx)
    wd = {kk: dev(torch, v) for kk, v in layer_weights(rng, ns).items()}
    x = rng.standard_normal((n_windows, n_ctx, ns)).astype(np.float32)
    got = dev(torch, x)
    scratch = torch.full((z.ops.encoder_layer_scratch(n_windows * n_ctx, ns),), float("nan"), device="cuda")
    ctx.encoder_layer_dev(got, n_windows, n_ctx, ns, n_head, wd, scratch)
    ref = dev(torch, x)
    composed_layer(torch, ctx, ref, n_windows, n_ctx, ns, n_head, wd)
    torch.cuda.synchronize()
    print(f"encoder layer images {n_windows}x{n_ctx}x{ns}/{n_head}: max abs diff "
          f"{float((got - ref).abs().max()):.2e}", flush=True)
    assert bool(torch.isfinite(got).all())
    assert torch.equal(got, ref)
