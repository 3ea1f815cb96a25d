"""GPU parity of the linear layers over seeded random shapes (zwg_linear_dev with f16 weights,
zwg_linear_q8_dev with int8 block weights, and zwg_linear_q8w_dev over the same weights uploaded
once and repacked).

Each case draws m (token steps, their tails, prefill rows), k (a multiple of 8, or of 32 for int8
blocks), n and whether there is a bias, so the kernels' tile tails, k splits and the choice
between the weight-streaming and tiled kernels all come up.  Outputs are checked against the f64
closed form over the f16 or dequantized weights (src/ops.zig:283-306, src/gemm.zig:274-351) at
the bar of the other linear tests, max abs <= 2e-5 * sqrt(k) on outputs of unit scale, for the
raw int8 call and the resident one alike.  (The two can split k differently, so they agree to
rounding; test_gpu_linear_q8.py holds them bit for bit at shapes where the splits coincide.)
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

N_CASES = 40


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


def draw(seed: int):
    rng = np.random.default_rng(seed)
    m = int(rng.choice([1, 2, 5, 17, 31, 32, 33, 63, 64, 65, 100, 256, 300, 777]))
    k_f16 = 8 * int(rng.integers(1, 384))
    k_q8 = 32 * int(rng.integers(1, 128))
    n = int(rng.integers(1, 3000))
    bias = bool(rng.integers(2))
    return rng, m, k_f16, k_q8, n, bias


def _ref(x, w, b):
    r = x.astype(np.float64) @ w.astype(np.float64).T
    return r if b is None else r + b.astype(np.float64)[None, :]


def _check(got, ref, k, what):
    err = float(np.abs(got - ref).max())
    bar = 2e-5 * np.sqrt(k)
    assert np.all(np.isfinite(got)) and err <= bar, f"{what}: max abs {err:.2e} (bar {bar:.1e})"


@pytest.mark.parametrize("seed", range(N_CASES))
def test_linear_fuzz(torch, ctx, seed):
    import zwhisper_amd as z

    rng, m, kf, kq, n, bias = draw(5100 + seed)
    print(f"case {seed}: m {m} k_f16 {kf} k_q8 {kq} n {n} bias {bias}", flush=True)
    b = rng.standard_normal(n).astype(np.float32) if bias else None
    bd = None if b is None else torch.from_numpy(b).cuda()

    x = rng.standard_normal((m, kf)).astype(np.float32)
    w = (rng.standard_normal((n, kf)) / np.sqrt(kf)).astype(np.float16)
    out = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_dev(torch.from_numpy(x).cuda(), m, kf, torch.from_numpy(w).cuda(), bd, n, out)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), _ref(x, w, b), kf, f"f16 {m}x{kf}x{n}")

    x = rng.standard_normal((m, kq)).astype(np.float32)
    wq = z.Q8.quantize((rng.standard_normal((n, kq)) / np.sqrt(kq)).astype(np.float16), n, kq)
    xd = torch.from_numpy(x).cuda()
    out = torch.full((m, n), float("nan"), device="cuda")
    ctx.linear_q8_dev(xd, m, kq, wq.to_device(), bd, n, out)
    torch.cuda.synchronize()
    raw = out.cpu().numpy()
    deq = oracle.q8_dequantize(wq.q, wq.scales)
    _check(raw, _ref(x, deq, b), kq, f"q8 {m}x{kq}x{n}")
    with wq.resident(ctx) as rw:
        out = torch.full((m, n), float("nan"), device="cuda")
        ctx.linear_q8w_dev(xd, m, rw, bd, out)
        torch.cuda.synchronize()
        res = out.cpu().numpy()
    # the packed path may split k differently from the raw one (at m <= 32 its workgroups cover
    # half as many weight rows), so the two agree to rounding, not always bit for bit
    _check(res, _ref(x, deq, b), kq, f"resident q8 {m}x{kq}x{n}")
    assert float(np.abs(res - raw).max()) <= 2e-5 * np.sqrt(kq), f"resident q8 {m}x{kq}x{n} far from the raw call"
