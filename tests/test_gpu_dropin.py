"""GPU tests of the host-pointer drop-in (zwg_attention_ex, the body of ops.attentionEx that the
unchanged callers bind, src/ops.zig:562-590): its device-side non-finite check on the split path,
and a context whose staging is fixed at zwg_open (zwg_limits.staging_bytes) so that no call
allocates, as the reference sizes its scratch once at load (src/ops.zig:545-560).

Bars as in tests/test_gpu_workloads.py: the f32 bar (max abs 2e-4, normwise rel 1e-3) for a
drop-in call, which the reference's own f32 attention meets (src/ops.zig:655-704 checks 1e-4
abs at its test shape).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import naive
from zwhisper_amd import workloads as W
from zwhisper_amd.ops import AttnShape

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_REL = 2e-4, 1e-3


@pytest.fixture(scope="module")
def torch():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    return torch


def check(got, ref, what, v_scale: float = 1.0):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = float(np.abs(got - ref).max())
    rel = err / max(float(np.abs(ref).max()), 1e-30)
    print(f"{what}: max abs {err:.2e}, normwise rel {rel:.2e}", flush=True)
    assert err <= TOL_ABS * max(v_scale, 1.0) and rel <= TOL_REL, f"{what}: {err:.3e} / {rel:.3e}"


def test_split_call_with_out_of_range_key_is_recomputed(torch):
    """A one-window tiny.en-sized call (1500 x 1500, 6 heads, non-causal) is split into key chunks and
    merged by the separate merge pass.  One key of magnitude 1e5 (beyond f16) makes the x3 kernel's
    rows of that head NaN; the merge sets the device flag, and the drop-in recomputes the call on the
    fp32 kernel, so the result meets the f32 bar against f64."""
    import zwhisper_amd as z

    n, h, d = 1500, 6, 64
    sh = AttnShape(n, n, h, h, d, h * d, h * d, h * d, False, None)
    assert z.plan(sh).max_chunks > 1, "the case must take the split path"
    q = W.normal(501, n * h * d)
    k = W.normal(502, n * h * d).reshape(n, h * d)
    k[777, 3 * d + 5] = 1.0e5  # head 3
    k = k.reshape(-1)
    v = W.normal(503, n * h * d)
    ref = naive.attention_f64(q, k, v, sh)
    with z.Context(0) as c:
        dev_out = torch.empty(n * h * d, device="cuda")
        c.attention_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh, dev_out)
        torch.cuda.synchronize()
        x3 = dev_out.cpu().numpy().reshape(n, h, d)
        assert np.isnan(x3[:, 3]).any(), "x3 device path: head 3 meets the out-of-range key"
        out = np.zeros(n * h * d, np.float32)
        c.attention_ex_host(q, k, v, sh, out)
    check(out, ref, "drop-in, split call with a key of 1e5")


def test_fixed_staging_serves_calls_within_it_and_refuses_beyond(torch):
    """zwg_limits.staging_bytes: the staging is allocated at zwg_open; a host call that fits runs and
    matches the device path bit for bit, a call that would need more staging is refused with an
    error naming staging_bytes (nothing is allocated), and the context stays usable after it."""
    import zwhisper_amd as z

    n, h, d = 1500, 6, 64  # q, k, v, out: 2.3 MB each
    sh = AttnShape(n, n, h, h, d, h * d, h * d, h * d, False, None)
    q, k, v = (W.normal(600 + i, n * h * d) for i in range(3))
    ref = naive.attention_f64(q, k, v, sh)
    with z.Context(0, staging_bytes=3 << 20) as c:
        out = np.zeros(n * h * d, np.float32)
        c.attention_ex_host(q, k, v, sh, out)
        check(out, ref, "fixed staging, 1500 x 384")
        dev_out = torch.empty(n * h * d, device="cuda")
        c.attention_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh, dev_out)
        torch.cuda.synchronize()
        assert np.array_equal(out, dev_out.cpu().numpy()), "drop-in and device path differ"
        hb = 12
        big = AttnShape(n, n, hb, hb, d, hb * d, hb * d, hb * d, False, None)  # 4.6 MB per tensor
        qb, kb, vb = (W.normal(700 + i, n * hb * d) for i in range(3))
        with pytest.raises(z.ZwgError, match="staging_bytes"):
            c.attention_ex_host(qb, kb, vb, big, np.zeros(n * hb * d, np.float32))
        out2 = np.zeros(n * h * d, np.float32)
        c.attention_ex_host(q, k, v, sh, out2)
        assert np.array_equal(out2, out)


def test_small_values_are_recomputed_in_fp32(torch):
    """Values of order 1e-5 (V scaled by 2^-17): the x3 kernel's f16 split of V has an absolute
    error floor near 2^-25, so on the device path its error stays at that floor while its relative
    error grows; the drop-in sees the small result (the kernels record its largest |value| on the
    device) and recomputes the call on the fp32 kernel, which meets the x3 bar relative to the
    result, as the reference's f32 attention would."""
    import zwhisper_amd as z

    n_q, n_kv, h, d = 200, 700, 4, 64
    sh = AttnShape(n_q, n_kv, h, h, d, h * d, h * d, h * d, True, None)
    q = W.normal(801, n_q * h * d)
    k = W.normal(802, n_kv * h * d)
    v = (W.normal(803, n_kv * h * d) * np.float32(2.0**-17)).astype(np.float32)
    ref = naive.attention_f64(q, k, v, sh)
    scale = float(np.abs(ref).max())
    with z.Context(0) as c:
        dev_out = torch.empty(n_q * h * d, device="cuda")
        c.attention_dev(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), sh, dev_out)
        torch.cuda.synchronize()
        err_dev = float(np.abs(dev_out.cpu().numpy().astype(np.float64) - ref).max())
        print(f"x3 device path, |V| ~ 2^-17: max abs {err_dev:.2e}, normwise rel {err_dev / scale:.2e}", flush=True)
        assert err_dev <= 2.0**-23, "the x3 error floor is absolute, near 2^-25"
        out = np.zeros(n_q * h * d, np.float32)
        c.attention_ex_host(q, k, v, sh, out)
    err = float(np.abs(out.astype(np.float64) - ref).max())
    print(f"drop-in, |V| ~ 2^-17: max abs {err:.2e}, normwise rel {err / scale:.2e}", flush=True)
    assert err / scale <= 3e-5, "the drop-in recomputes a small result on the fp32 kernel"
