"""GPU parity of the linear layer (zwg_linear / zwg_linear_dev, f16 weights) against the f64
closed form and the oracle's ops.linear (src/ops.zig:283-306).

Bar: max abs error <= 2e-5 * sqrt(k) on outputs of unit scale (x ~ N(0, 1), w ~ N(0, 1/k)), the
size of the reference's own f32 accumulation error, and never worse than the oracle by more
than that.  Known answers: with identity or one-hot weights every output is exactly the two-term
split's value, f32(w*hi + w*lo) with hi = f16(x), lo = f16(x - hi) -- which keeps 22 of f32's 24
significand bits of x.
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
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float32) if bias else None
    return x, w, b


def run_dev(torch, ctx, x, w, b, m, k, n):
    out = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_dev(torch.from_numpy(x).cuda(), m, k, torch.from_numpy(w).cuda(),
                   None if b is None else torch.from_numpy(b).cuda(), n, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def ref64(x, w, b):
    r = x.astype(np.float64) @ w.astype(np.float64).T
    return r if b is None else r + b.astype(np.float64)[None, :]


@pytest.mark.parametrize("m,k,n", [
    (1500, 384, 384),    # tiny.en Q/K/V/O (src/encoder.zig:164-168)
    (1500, 384, 1536),   # tiny.en MLP up (:172)
    (1500, 1536, 384),   # tiny.en MLP down (:174)
    (1500, 512, 512),    # base.en projections
    (3000, 240, 384),    # conv1 as a linear over im2col rows, k = 80 mels x 3 (:139)
    (7, 8, 5), (1, 64, 1), (65, 72, 130), (129, 520, 257),  # tails in m, n and k
])
def test_linear_matches_reference(torch, ctx, m, k, n):
    x, w, b = inputs(m * 7 + n, m, k, n)
    got = run_dev(torch, ctx, x, w, b, m, k, n)
    ref = ref64(x, w, b)
    err = float(np.abs(got - ref).max())
    bar = 2e-5 * np.sqrt(k)
    print(f"linear {m}x{k}x{n}: max abs {err:.2e} (bar {bar:.1e})", flush=True)
    assert np.all(np.isfinite(got)) and err <= bar
    if m * n * k <= 50_000_000:
        with oracle.Oracle(4) as o:
            ora = o.linear_f16(x, m, k, w, b, n).reshape(m, n)
        assert float(np.abs(got - ora).max()) <= err + bar


@pytest.mark.parametrize("m,k,n", [
    (24033, 1000, 1288),  # the 128 x 256 tiles: a partial row tile, a partial column tile, k % 32 = 8
    (8200, 264, 520),     # the 64 x 256 tiles, the same tails
])
def test_linear_large_tiles(torch, ctx, m, k, n):
    """Shapes large enough for the x 256 tiles (the encoder's 16-window projections take them),
    with tails in every dimension, against f64."""
    x, w, b = inputs(m + 3 * n + k, m, k, n)
    got = run_dev(torch, ctx, x, w, b, m, k, n)
    ref = ref64(x, w, b)
    err = float(np.abs(got - ref).max())
    bar = 2e-5 * np.sqrt(k)
    print(f"linear {m}x{k}x{n}: max abs {err:.2e} (bar {bar:.1e})", flush=True)
    assert np.all(np.isfinite(got)) and err <= bar


def split_product(x, wv):
    """What one weight times x gives through the two-term split: f32(wv*hi + wv*lo), hi = f16(x),
    lo = f16(x - hi) -- both products exact in f32, one rounding for the sum."""
    hi = x.astype(np.float16).astype(np.float32)
    lo = (x - hi).astype(np.float16).astype(np.float32)
    w = np.float32(wv)
    return (w * hi + w * lo).astype(np.float32)


def test_identity_and_one_hot(torch, ctx):
    """With one nonzero weight per output, the result is exactly the split's value."""
    m, k = 300, 64
    x = np.random.default_rng(1).standard_normal((m, k)).astype(np.float32)
    x[0, :8] = [1e-4, -3e-5, 7e-8, 65000.0, -1.0, 0.0, 1.0 / 3.0, 2.0 ** -14]  # subnormal lo, large, exact
    got = run_dev(torch, ctx, x, np.eye(k, dtype=np.float16), None, m, k, k)
    assert np.array_equal(got, split_product(x, 1.0))
    assert np.max(np.abs(got - x) / np.maximum(np.abs(x), 2.0 ** -4)) <= 2.0 ** -21
    w = np.zeros((2, k), np.float16)
    w[0, 3] = 1
    w[1, 63] = -2
    got = run_dev(torch, ctx, x, w, None, m, k, 2)
    assert np.array_equal(got[:, 0], split_product(x[:, 3], 1.0))
    assert np.array_equal(got[:, 1], split_product(x[:, 63], -2.0))


def test_host_dropin(torch, ctx):
    """zwhisper_amd.linear: ops.linear's call form on host arrays."""
    import zwhisper_amd as z

    m, k, n = 200, 128, 96
    x, w, b = inputs(9, m, k, n)
    out = np.zeros(m * n, np.float32)
    z.linear(None, x.reshape(-1), m, k, w, b, n, out)
    assert float(np.abs(out.reshape(m, n) - ref64(x, w, b)).max()) <= 2e-5 * np.sqrt(k)


def test_large_input_turns_inf_not_wrong(torch, ctx):
    """An input beyond f16's range makes its output row non-finite rather than silently wrong."""
    m, k, n = 4, 16, 8
    x, w, _ = inputs(3, m, k, n, bias=False)
    x[2, 5] = 1e6
    got = run_dev(torch, ctx, x, w, None, m, k, n)
    assert not np.all(np.isfinite(got[2]))
    assert np.all(np.isfinite(got[[0, 1, 3]]))


def test_linear_errors(torch, ctx):
    import zwhisper_amd as z

    t = torch.zeros(64, device="cuda")
    w = torch.zeros(64, dtype=torch.float16, device="cuda")
    with pytest.raises(z.ZwgError, match="multiple of 8"):
        ctx.linear_dev(t, 2, 12, w, None, 2, t)
    with pytest.raises(z.ZwgError, match="float16"):
        ctx.linear_dev(t, 2, 8, t, None, 2, t)


# Large calls run 64 x 256 (or 128 x 256) tiles, small ones 64 x 64; every tile shape accumulates
# each output over k in the same order (stages of 32 k in order, per 16-k step the hi then the lo
# product), so a row computed in a large unsplit call equals the same row computed in a small
# unsplit call bit for bit.  Shapes: the base.en projections' width, an n with a partial column
# tile, m and n tails with 3 stages of k, and 5 stages.
TILE_CASES = [(16384, 256, 512), (12000, 448, 768), (8193, 96, 1040), (16400, 160, 256)]


@pytest.mark.parametrize("m,k,n", TILE_CASES)
def test_large_and_small_calls_agree_bitwise(torch, ctx, m, k, n):
    from zwhisper_amd import _lib

    x, w, b = inputs(m + k + n, m, k, n)
    xd, wd, bd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda()
    big = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_epi_dev(xd, m, k, wd, bd, n, big, _lib.EPI_NONE)
    gel = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_epi_dev(xd, m, k, wd, bd, n, gel, _lib.EPI_GELU)
    wide = torch.full((m, 2 * n), 7.0, device="cuda")
    ctx.linear_epi_dev(xd, m, k, wd, bd, n, wide.view(-1)[n:], _lib.EPI_NONE, out_stride=2 * n)
    torch.cuda.synchronize()
    got = big.cpu().numpy()
    ref = ref64(x, w, b)
    err = float(np.abs(got - ref).max())
    print(f"linear {m}x{k}x{n}: max abs {err:.2e}", flush=True)
    assert np.all(np.isfinite(got)) and err <= 2e-5 * np.sqrt(k)
    ref_g = big.clone()
    ctx.gelu_dev(ref_g)
    torch.cuda.synchronize()
    assert torch.equal(gel, ref_g)
    assert torch.equal(wide[:, n:], big) and bool((wide[:, :n] == 7.0).all())
    for r0, r1 in ((0, 64), (m - 61, m), (4999, 5130)):
        small = torch.full((r1 - r0, n), float("nan"), device="cuda")
        ctx.linear_epi_dev(xd[r0:r1].contiguous(), r1 - r0, k, wd, bd, n, small, _lib.EPI_NONE)
        torch.cuda.synchronize()
        assert torch.equal(small, big[r0:r1]), (r0, r1)
