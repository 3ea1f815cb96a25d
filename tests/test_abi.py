"""The C ABI library on a machine without a GPU: it loads, exports what include/zw_gpu.h
declares, checks shapes and plans calls the way its callers rely on, and fails cleanly when no
device is present.  No compute call is made here.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import pytest

import zwhisper_amd as z
from zwhisper_amd import _lib
from zwhisper_amd.ops import AttnShape

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def gpu_present() -> bool:
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


def test_library_is_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run `python -m zwhisper_amd.build` first"
    L = _lib.lib()
    assert L.zwg_version() == 2


def test_every_declared_symbol_is_exported():
    declared = _lib.declared_symbols()
    assert len(declared) >= 13
    L = _lib.lib()
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/zw_gpu.h but not exported"
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in nm.stdout.splitlines() if line.strip()}
    assert set(declared) <= exported


def test_cpp_mirror_symbols_exported():
    nm = subprocess.run(["nm", "-DC", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    for sym in ("zw::ops::attentionEx(", "zw::ops::attention(", "zw::ops::attentionScratchEx(",
                "zw::ops::attentionScratchKT(", "zw::ops::attentionScratch("):
        assert sym in nm.stdout, sym


def test_header_compiles_as_c():
    """include/zw_gpu.h is plain C (no C++ in the signatures)."""
    src = '#include "zw_gpu.h"\nint main(void){zwg_attn_shape s={0}; (void)s; return 0;}\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        "-x", "c", "-"], input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_struct_layout_matches_header():
    assert ctypes.sizeof(_lib.ShapeC) == 9 * 8 + 2 * 4
    assert ctypes.sizeof(_lib.BatchC) == 6 * 8
    assert ctypes.sizeof(_lib.PlanC) == 2 * 4 + 4 * 8
    assert ctypes.sizeof(_lib.LimitsC) == 8 + 2 * 4 + 8


def S(n_q, n_kv, h, hkv, d, causal, kt=None, qs=None, kvs=None, os_=None):
    return AttnShape(n_q, n_kv, h, hkv, d, qs or h * d, kvs or hkv * d, os_ or h * d, causal, kt)


@pytest.mark.parametrize("sh", [
    S(1500, 1500, 6, 6, 64, False, kt=1504), S(1, 448, 12, 12, 64, True), S(2048, 2048, 14, 2, 64, True, kt=2048),
    S(1, 4096, 12, 2, 128, True, kt=4096), S(20, 20, 12, 12, 32, False), S(0, 0, 1, 1, 64, False),
    S(3, 0, 2, 2, 64, False), S(2, 3, 2, 2, 48, False), S(2, 3, 2, 2, 16, False), S(5, 9, 4, 2, 4, True, kt=12),
    S(7, 7, 2, 1, 100, False), S(3, 5, 2, 1, 132, True), S(3, 5, 2, 2, 256, False), S(1, 9, 1, 1, 1024, False),
])
def test_check_shape_accepts(sh):
    z.check_shape(sh)


@pytest.mark.parametrize("sh,msg", [
    (S(2, 3, 2, 2, 50, False), "head dim"),
    (S(2, 3, 2, 2, 1028, False), "head dim"),
    (S(2, 3, 2, 2, 134, False), "head dim"),
    (S(2, 3, 2, 2, 0, False), "head dim"),
    (S(2, 3, 3, 2, 64, False), "multiple of n_head_kv"),
    (S(2, 3, 0, 1, 64, False), "multiple of n_head_kv"),
    (S(4, 3, 2, 2, 64, True), "n_kv >= n_q"),
    (S(2, 3, 2, 2, 64, False, qs=130), "multiples of 4"),
    (S(2, 3, 2, 2, 64, False, qs=64), "q_stride is smaller"),
    (S(2, 3, 2, 2, 64, False, os_=64), "out_stride is smaller"),
    (S(2, 3, 2, 2, 64, False, kvs=64), "kv_stride is smaller"),
    (S(2, 30, 2, 2, 64, False, kt=16), "kt_stride is smaller"),
])
def test_check_shape_rejects(sh, msg):
    with pytest.raises(z.ZwgError, match=msg):
        z.check_shape(sh)


def test_reserved_field_must_be_zero():
    c = S(1, 1, 1, 1, 64, False).to_c()
    c.reserved = 1
    buf = ctypes.create_string_buffer(128)
    assert _lib.lib().zwg_check_shape(ctypes.byref(c), buf, 128) == _lib.ZWG_ERROR
    assert b"reserved" in buf.value


# ---------------------------------------------------------------------------------------------
# planning (which kernel, how keys are split)


def test_plan_picks_the_f32_kernel_above_128():
    """Head dims above the built kernels' 128 run on the plain f32 kernel, one wavefront per query
    row, unsplit, with no workspace."""
    for sh, nb in ((S(1500, 1500, 2, 2, 256, False), 1), (S(1, 300, 8, 2, 192, True, kt=304), 4)):
        p = z.plan(sh, nb)
        assert p.kernel == 3 and p.max_chunks == 1 and p.workspace_bytes == 0
        assert p.grid_blocks == -(-nb * sh.n_head * sh.n_q // 4)


def test_plan_picks_decode_for_few_rows_per_kv_head():
    assert z.plan(S(1, 448, 12, 12, 64, True), 32).kernel == 2        # Whisper decoder step
    assert z.plan(S(1, 4096, 12, 2, 128, True, kt=4096), 64).kernel == 2  # GQA 6 rows
    assert z.plan(S(1, 4096, 14, 2, 64, True, kt=4096)).kernel == 2   # GQA 7 rows
    assert z.plan(S(4, 33, 4, 2, 64, True)).kernel == 2               # 2 queries x 2 heads
    assert z.plan(S(2, 33, 14, 2, 64, True)).kernel == 1              # 14 rows: dense kernel
    assert z.plan(S(1500, 1500, 6, 6, 64, False, kt=1504)).kernel == 1


def unit_split(kv_hi, tile, chunk_len, max_chunks):
    """The kernels' key split of one work unit (attn_kernels.hpp, unit_split): (chunks, keys each)."""
    w = -(-kv_hi // tile)
    if w <= 0:
        return 1, tile
    tau = max(1, chunk_len // tile)
    nc = min(max((w + tau // 2) // tau, 1), max_chunks)
    lt = -(-w // nc)
    return -(-w // lt), lt * tile


@pytest.mark.parametrize("sh,nb", [
    (S(1500, 1500, 6, 6, 64, False, kt=1504), 1), (S(1500, 1500, 8, 8, 64, False, kt=1504), 16),
    (S(2048, 2048, 14, 2, 64, True, kt=2048), 1), (S(1, 4096, 12, 2, 128, True, kt=4096), 64),
    (S(1, 1500, 12, 12, 64, False), 32), (S(1, 448, 12, 12, 64, True), 32), (S(70, 90, 2, 2, 32, True), 1),
])
def test_plan_invariants(sh, nb):
    p = z.plan(sh, nb)
    # decode: 256-key tiles, or 64 for row-major caches of at most 512 keys; dense: 32
    tile = (64 if not sh.kt_stride and sh.n_kv <= 512 else 256) if p.kernel == 2 else 32
    assert p.chunk_len % tile == 0 and p.chunk_len > 0
    # every unit's keys are covered by at most max_chunks non-empty chunks
    his = ([sh.n_kv - sh.n_q + min(sh.n_q, (qb + 1) * 128) if sh.causal else sh.n_kv
            for qb in range(-(-sh.n_q // 128))] if p.kernel == 1 else list(range(0, sh.n_kv + 1, 7)) + [sh.n_kv])
    for hi in his:
        n, keys = unit_split(hi, tile, p.chunk_len, p.max_chunks)
        assert 1 <= n <= p.max_chunks
        assert keys % tile == 0 and (n - 1) * keys < max(hi, 1) <= n * keys or hi == 0
    rows = nb * sh.n_head * sh.n_q
    # (max, sum) pairs, then the sums from the next 256-byte boundary (aligned 16-byte accesses)
    pairs = -(-(2 * rows * p.max_chunks) // 64) * 64
    assert p.workspace_bytes == ((pairs + rows * p.max_chunks * sh.d) * 4 if p.max_chunks > 1 else 0)
    if p.kernel == 2:
        assert p.grid_blocks == p.max_chunks * sh.n_head_kv * nb
    elif sh.causal:
        # causal dense calls launch only the (q-block, chunk, head) triples that have keys
        live = sum(unit_split(sh.n_kv - sh.n_q + min(sh.n_q, (qb + 1) * 128), tile, p.chunk_len, p.max_chunks)[0]
                   for qb in range(-(-sh.n_q // 128)))
        assert p.grid_blocks == live * sh.n_head * nb
    else:
        assert p.grid_blocks == p.max_chunks * -(-sh.n_q // 128) * sh.n_head * nb


def test_plan_headline_encoder_is_not_split():
    p = z.plan(S(1500, 1500, 8, 8, 64, False, kt=1504), 16)
    assert p.kernel == 1 and p.max_chunks == 1 and p.workspace_bytes == 0


def test_plan_respects_a_small_workspace():
    sh = S(1, 4096, 12, 2, 128, True, kt=4096)
    big = z.plan(sh, 64)
    assert big.max_chunks > 1
    small = z.plan(sh, 64, workspace_bytes=big.workspace_bytes // 4)
    assert small.max_chunks < big.max_chunks
    assert 0 < small.workspace_bytes <= big.workspace_bytes // 4
    none = z.plan(sh, 64, workspace_bytes=1)
    assert none.max_chunks == 1 and none.workspace_bytes == 0


# ---------------------------------------------------------------------------------------------
# the Python mirror of the ops interface


def test_scratch_sizes_follow_the_reference():
    # src/ops.zig:545-560 at the tiny.en encoder shape: n_kv_pad = 1504, 24 q-blocks
    assert z.attentionScratch(1500, 1500, 6, 384) == 6 * 64 * 1504 + 6 * 24 * 64 * 1504
    assert z.attentionScratchEx(1, 300, 12, 2, 128) == 2 * 128 * 304 + 12 * 1 * 64 * 304
    assert z.attentionScratchKT(256, 4096, 14) == 14 * 4 * 64 * 4096
    assert z.q_block == 64 and z.V == 16


def test_shape_extents():
    sh = S(3, 5, 4, 2, 64, True, kt=8, qs=300, kvs=132, os_=260)
    assert sh.q_len() == 2 * 300 + 256
    assert sh.out_len() == 2 * 260 + 256
    assert sh.k_len() == (2 * 64 - 1) * 8 + 5
    assert sh.v_len() == 4 * 132 + 128


@pytest.mark.skipif(gpu_present(), reason="checks the no-device error path")
def test_open_without_device_fails_cleanly():
    with pytest.raises(z.ZwgError, match="no HIP device"):
        z.Context(0)


@pytest.mark.skipif(gpu_present(), reason="checks the no-device error path")
def test_python_mirror_raises_like_a_failed_assert():
    import numpy as np

    q = np.zeros(64, np.float32)
    out = np.zeros(64, np.float32)
    with pytest.raises(z.ZwgError):
        z.attention(None, q, q, q, 1, 1, 64, 1, False, None, out)


def test_mirror_rejects_non_f32_buffers():
    import numpy as np

    with pytest.raises(z.ZwgError, match="float32"):
        z.attentionEx(None, np.zeros(64), np.zeros(64, np.float32), np.zeros(64, np.float32),
                      S(1, 1, 1, 1, 64, False), None, np.zeros(64, np.float32))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_noalloc_refuses_beyond_its_scratch_before_the_device():
    """zwg_attention_batch_noalloc checks the call's split partials against its static scratch
    before it touches a device: a too-large call fails with that reason, GPU or not."""
    import ctypes

    sh = S(2048, 2048, 32, 32, 128, True)
    assert z.plan(sh).workspace_bytes > _lib.NOALLOC_SCRATCH_BYTES
    c = sh.to_c()
    fake = 1 << 20  # an aligned, never dereferenced address
    rc = _lib.lib().zwg_attention_batch_noalloc(fake, fake, fake, ctypes.byref(c), None, fake, 0, None)
    assert rc == _lib.ZWG_ERROR
    assert "static scratch" in _lib.last_error(None)


@pytest.mark.parametrize("dense_math", [0, 1])
def test_dense_k_v_spans_beyond_2gib_are_refused_in_both_modes(dense_math):
    """Both dense kernels (x3 and fp32) address an item's K/V rows with 32-bit buffer offsets, so a
    call whose rows span 2 GiB or more is refused with that reason before any device work: an
    unsplit (512 units) non-causal call with a 1 GiB row stride, through the entry point that
    needs no context."""
    import ctypes

    n_q = 128 * 512
    sh = AttnShape(n_q, 2, 1, 1, 64, 64, 1 << 28, 64, False, None)
    assert z.plan(sh).max_chunks == 1 and z.plan(sh).kernel == 1
    c = sh.to_c()
    fake = 1 << 20  # an aligned, never dereferenced address
    rc = _lib.lib().zwg_attention_batch_noalloc(fake, fake, fake, ctypes.byref(c), None, fake, dense_math, None)
    assert rc == _lib.ZWG_ERROR
    assert "2 GiB" in _lib.last_error(None)
    # the transposed-K span of one KV head: d rows of kt_stride columns
    sh = AttnShape(n_q, 2, 1, 1, 64, 64, 64, 64, False, 1 << 23)
    c = sh.to_c()
    rc = _lib.lib().zwg_attention_batch_noalloc(fake, fake, fake, ctypes.byref(c), None, fake, dense_math, None)
    assert rc == _lib.ZWG_ERROR
    assert "transposed K rows" in _lib.last_error(None)


def test_zig_binding_declares_the_whole_header():
    """zig/gpu.zig (the binding a maintainer drops into src/gpu.zig; no Zig toolchain here to
    compile it) declares every function of include/zw_gpu.h, and its extern structs carry the C
    structs' fields in the same order."""
    import re

    text = open(os.path.join(ROOT, "zig", "gpu.zig")).read()
    zig_fns = sorted(set(re.findall(r'pub extern "zwgpu" fn (zwg_[a-z_0-9]+)\(', text)))
    assert zig_fns == _lib.declared_symbols()

    def zig_fields(name):
        body = re.search(r"pub const %s = extern struct \{(.*?)\n\};" % name, text, re.S).group(1)
        return re.findall(r"^\s+([a-z_0-9]+):", body, re.M)

    for zname, cstruct in (("Shape", _lib.ShapeC), ("Batch", _lib.BatchC), ("Limits", _lib.LimitsC),
                           ("PlanInfo", _lib.PlanC), ("KvDesc", _lib.KVDescC), ("KvInfo", _lib.KVInfoC),
                           ("EncLayer", _lib.EncLayerC), ("DecLayer", _lib.DecLayerC), ("Decoder", _lib.DecoderC),
                           ("LlmLayer", _lib.LlmLayerC), ("Llm", _lib.LlmC)):
        assert zig_fields(zname) == [f for f, _ in cstruct._fields_], zname
