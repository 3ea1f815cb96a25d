"""GPU parity: the HIP path (through the C ABI) against the f64 closed form and the CPU oracle.

Tolerances, by the arithmetic of the context (include/zw_gpu.h states the same):
  * fp32 dense mode and the decode kernels -- the reference's f32 attention bar: max |gpu - ref|
    <= 2e-4 and normwise relative error ||gpu - ref||_inf / ||ref||_inf <= 1e-3;
  * the x3 dense mode (the default; split 16-bit MFMA products) -- its own bar: max abs <= 5e-5
    and normwise relative <= 3e-5.  A context in x3 mode is held to it for every call, its decode
    calls (f32 FMA, ~1e-7) included.
The elementwise relative error over outputs with |ref| >= 1e-2 is printed beside them (reported,
no bound of its own).  Columns a call must not write (row gaps when out_stride > n_head * d) must
keep their previous contents.
"""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

from _golden import head_columns_mask, load_cases

pytestmark = pytest.mark.gpu

TOL_ABS = 2e-4  # f32 bar
TOL_REL = 1e-3
TOL_ABS_X3 = 5e-5  # x3 dense mode
TOL_REL_X3 = 3e-5
SENTINEL = 7.25

CASES = load_cases()
CASE_IDS = [c.name for c in CASES]


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


def assert_close(got: np.ndarray, ref: np.ndarray, what: str, x3: bool = True) -> tuple[float, float]:
    """Max abs and normwise relative error of got against ref, held to the x3 bar (x3=True) or
    the f32 bar."""
    tol_abs, tol_rel = (TOL_ABS_X3, TOL_REL_X3) if x3 else (TOL_ABS, TOL_REL)
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    if ref.size == 0:
        return 0.0, 0.0
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = float(np.abs(got - ref).max())
    rel = err / max(float(np.abs(ref).max()), 1e-30)
    big = np.abs(ref) >= 1e-2
    erel = float((np.abs(got - ref)[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    print(f"{what}: max abs {err:.3e}, normwise rel {rel:.3e}, elementwise rel (|ref| >= 1e-2) {erel:.3e}",
          flush=True)
    assert err <= tol_abs and rel <= tol_rel, (f"{what}: max abs {err:.3e} (<= {tol_abs}), normwise rel {rel:.3e} "
                                               f"(<= {tol_rel})")
    return err, rel


def to_dev(torch, a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32).reshape(-1)).cuda()


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_golden_device_pointers(torch, ctx, case):
    print(f"case {case.name} shape={case.shape}", flush=True)
    sh = case.shape
    q, k, v = to_dev(torch, case.q), to_dev(torch, case.k), to_dev(torch, case.v)
    out = torch.full((max(sh.out_len(), 1),), SENTINEL, dtype=torch.float32, device="cuda")
    ctx.attention_dev(q, k, v, sh, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    m = head_columns_mask(sh)
    assert_close(got[m], case.expected[m], case.name)
    assert np.all(got[~m] == SENTINEL), f"{case.name}: wrote outside the head columns"


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_golden_dense_fp32_mode(torch, ctx_fp32, case):
    """The same golden cases with the dense calls on the fp32-MFMA kernel (ZWG_DENSE_FP32)."""
    print(f"case {case.name} (fp32 dense)", flush=True)
    sh = case.shape
    q, k, v = to_dev(torch, case.q), to_dev(torch, case.k), to_dev(torch, case.v)
    out = torch.full((max(sh.out_len(), 1),), SENTINEL, dtype=torch.float32, device="cuda")
    ctx_fp32.attention_dev(q, k, v, sh, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    m = head_columns_mask(sh)
    assert_close(got[m], case.expected[m], case.name, x3=False)
    assert np.all(got[~m] == SENTINEL), f"{case.name}: wrote outside the head columns"


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_golden_host_dropin(ctx, case):
    """zwg_attention_ex: host pointers, synchronous (the ops.attentionEx drop-in)."""
    print(f"case {case.name} (host)", flush=True)
    sh = case.shape
    out = np.full(max(sh.out_len(), 1), SENTINEL, dtype=np.float32)
    ctx.attention_ex_host(case.q, case.k, case.v, sh, out)
    m = head_columns_mask(sh)
    if case.expected.size:
        assert_close(out[m], case.expected[m], case.name)
    assert np.all(out[~m] == SENTINEL), f"{case.name}: wrote outside the head columns"


def test_cpp_mirror_parity(torch):
    """The C++ mirror of ops.attention/attentionEx, tested like src/ops.zig:655-704."""
    from zwhisper_amd import build

    exe = build.CPP_TEST_BIN
    assert os.path.exists(exe), "tests/cpp/test_attention.cpp is not built (python -m zwhisper_amd.build)"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_golden_vs_oracle_agree_on_gpu_inputs(torch, ctx):
    """The oracle and the GPU agree with each other on the reference test's shape."""
    import oracle

    case = next(c for c in CASES if c.name == "ref_test_causal")
    o = oracle.Oracle(2)
    ref = o.attention_ex(case.q, case.k, case.v, case.shape)
    out = np.zeros(case.shape.out_len(), dtype=np.float32)
    ctx.attention_ex_host(case.q, case.k, case.v, case.shape, out)
    assert_close(out, ref, "gpu vs oracle")
    o.close()
