"""Python mirror of zwhisper's attention interface (src/ops.zig:464-605) on the gfx950 library.

Same names and argument meaning as the Zig module:

* ``q_block``, ``V`` (src/ops.zig:473, src/gemm.zig:15-24);
* ``AttnShape`` (src/ops.zig:477-492), ``kt_stride=None`` for row-major keys;
* ``attentionScratchEx`` / ``attentionScratchKT`` / ``attentionScratch`` (src/ops.zig:545-560);
* ``attentionEx(pool, q, k, v, sh, scratch, out)`` and
  ``attention(pool, q, k, v, n_q, n_kv, n_state, n_head, causal, scratch, out)`` on host
  (numpy float32) buffers: synchronous, `out` complete on return, only each row's
  n_head*d columns written (src/ops.zig:540).

Where the reference asserts (src/ops.zig:564, :568) these raise ``ZwgError``.  ``pool`` and
``scratch`` are accepted and unused.  ``Context`` adds the device-pointer calls (torch CUDA
tensors already in HBM, on torch's current stream) that the benchmarks and batched callers use.
"""
from __future__ import annotations

import ctypes
import threading
import weakref
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import ZwgError

V = 16
q_block = 64


@dataclass(frozen=True)
class AttnShape:
    n_q: int
    n_kv: int
    n_head: int
    n_head_kv: int
    d: int
    q_stride: int
    kv_stride: int
    out_stride: int
    causal: bool
    kt_stride: Optional[int] = None

    def to_c(self) -> _lib.ShapeC:
        return _lib.ShapeC(self.n_q, self.n_kv, self.n_head, self.n_head_kv, self.d, self.q_stride, self.kv_stride,
                           self.out_stride, self.kt_stride or 0, 1 if self.causal else 0, 0)

    # extents (in floats) the reference reads or writes
    def q_len(self) -> int:
        return (self.n_q - 1) * self.q_stride + self.n_head * self.d if self.n_q else 0

    def out_len(self) -> int:
        return (self.n_q - 1) * self.out_stride + self.n_head * self.d if self.n_q else 0

    def k_len(self) -> int:
        if self.n_kv == 0:
            return 0
        kvd = self.n_head_kv * self.d
        if self.kt_stride:
            return (kvd - 1) * self.kt_stride + self.n_kv
        return (self.n_kv - 1) * self.kv_stride + kvd

    def v_len(self) -> int:
        return (self.n_kv - 1) * self.kv_stride + self.n_head_kv * self.d if self.n_kv else 0


def attentionScratchEx(n_q: int, n_kv: int, n_head: int, n_head_kv: int, d: int) -> int:
    n_kv_pad = (n_kv + V - 1) // V * V
    n_qblocks = (n_q + q_block - 1) // q_block
    return n_head_kv * d * n_kv_pad + n_head * n_qblocks * q_block * n_kv_pad


def attentionScratchKT(n_q: int, kt_stride: int, n_head: int) -> int:
    n_qblocks = (n_q + q_block - 1) // q_block
    return n_head * n_qblocks * q_block * kt_stride


def attentionScratch(n_q: int, n_kv: int, n_head: int, n_state: int) -> int:
    return attentionScratchEx(n_q, n_kv, n_head, n_head, n_state // n_head)


def check_shape(sh: AttnShape) -> None:
    """Raises ZwgError with the library's message if `sh` is not accepted."""
    buf = ctypes.create_string_buffer(256)
    c = sh.to_c()
    if _lib.lib().zwg_check_shape(ctypes.byref(c), buf, 256) != _lib.ZWG_OK:
        raise ZwgError(buf.value.decode())


def plan(sh: AttnShape, n_batch: int = 1, workspace_bytes: int = 0) -> _lib.PlanC:
    """Which kernel and key split a call would use (host-only)."""
    c = sh.to_c()
    b = _lib.BatchC(n_batch, 0, 0, 0, 0, None)
    p = _lib.PlanC()
    _lib.check(_lib.lib().zwg_plan(ctypes.byref(c), ctypes.byref(b), workspace_bytes, ctypes.byref(p)))
    return p


class Context:
    """One library context (zwg_ctx): a device, a workspace, staging buffers."""

    def __init__(self, device: int = 0, workspace_bytes: int = 0, dense_math: int = 0, staging_bytes: int = 0):
        """dense_math: _lib.DENSE_X3 (0, default) or _lib.DENSE_FP32, the dense kernel's arithmetic.
        staging_bytes: non-zero allocates every staging buffer at this size now, and calls that
        would need more are refused (zwg_limits.staging_bytes)."""
        L = _lib.lib()
        self._L = L
        h = ctypes.c_void_p()
        lim = _lib.LimitsC(workspace_bytes, dense_math, 0, staging_bytes)
        rc = L.zwg_open(device, ctypes.byref(lim), ctypes.byref(h))
        if rc != _lib.ZWG_OK:
            raise ZwgError(_lib.last_error(None))
        self._h = h
        self.device = device
        # objects made from this context (KVCache, Q8Resident): closed before the context is
        self._children = weakref.WeakSet()

    def _adopt(self, child) -> None:
        self._children.add(child)

    def set_dense_math(self, mode: int) -> None:
        """Switch the dense kernel's arithmetic (_lib.DENSE_X3 or _lib.DENSE_FP32) for later calls."""
        self._check(self._L.zwg_set_dense_math(self._h, mode))

    def close(self) -> None:
        if getattr(self, "_h", None):
            for child in list(getattr(self, "_children", ())):
                child.close()
            self._L.zwg_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        if not self._h:
            raise ZwgError("the context is closed")
        return self._h

    def _check(self, rc: int) -> None:
        if rc != _lib.ZWG_OK:
            raise ZwgError(_lib.last_error(self._h))

    def set_stream(self, stream_ptr: int | None) -> None:
        self._check(self._L.zwg_set_stream(self._h, stream_ptr))

    def sync(self) -> None:
        self._check(self._L.zwg_sync(self._h))

    # ---- host buffers: the drop-in
    def attention_ex_host(self, q: np.ndarray, k: np.ndarray, v: np.ndarray, sh: AttnShape, out: np.ndarray) -> None:
        for name, a in (("q", q), ("k", k), ("v", v), ("out", out)):
            if a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]:
                raise ZwgError(f"{name} must be a contiguous float32 array")
        if q.size < sh.q_len() or out.size < sh.out_len() or k.size < sh.k_len() or v.size < sh.v_len():
            raise ZwgError("a buffer is shorter than the shape needs")
        c = sh.to_c()
        self._check(self._L.zwg_attention_ex(self._h, q.ctypes.data, k.ctypes.data, v.ctypes.data, ctypes.byref(c),
                                             out.ctypes.data))

    # ---- device buffers (torch CUDA tensors, float32), on torch's current stream
    def _bind_torch_stream(self):
        import torch

        self.set_stream(torch.cuda.current_stream(self.device).cuda_stream)

    @staticmethod
    def _dev_ptr(t, name: str) -> int:
        import torch

        if t is None:
            return 0
        if isinstance(t, int):  # a raw device address (e.g. a KVCache's cache pointers)
            return t
        if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32:
            raise ZwgError(f"{name} must be a CUDA float32 tensor")
        return t.data_ptr()

    def linear_dev(self, x, m: int, k: int, w, bias, n: int, out) -> None:
        """out[m][n] = x[m][k] . w[n][k]^T (+ bias): CUDA tensors, x/bias/out float32, w float16."""
        import torch

        if not isinstance(w, torch.Tensor) or not w.is_cuda or w.dtype != torch.float16:
            raise ZwgError("w must be a CUDA float16 tensor")
        if x.numel() < m * k or w.numel() < n * k or out.numel() < m * n or (bias is not None and bias.numel() < n):
            raise ZwgError("a tensor is shorter than m, n and k need")
        self._bind_torch_stream()
        self._check(self._L.zwg_linear_dev(self._h, self._dev_ptr(x, "x"), m, k, w.data_ptr(), _lib.W_F16,
                                           self._dev_ptr(bias, "bias"), n, self._dev_ptr(out, "out")))

    def linear_q8_dev(self, x, m: int, k: int, w: "Q8", bias, n: int, out) -> None:
        """out[m][n] = x[m][k] . dequant(w)^T (+ bias) over int8 block weights: CUDA tensors, w.q int8
        [n][k] and w.scales float32 [n][k / 32] (see Q8.to_device), x/bias/out float32."""
        import torch

        if not isinstance(w, Q8) or not isinstance(w.q, torch.Tensor) or not w.q.is_cuda or w.q.dtype != torch.int8:
            raise ZwgError("w must be a Q8 holding CUDA tensors (Q8.to_device)")
        if w.n != n or w.k != k:
            raise ZwgError(f"w is [{w.n}][{w.k}], the call asks for [{n}][{k}]")
        if x.numel() < m * k or out.numel() < m * n or (bias is not None and bias.numel() < n):
            raise ZwgError("a tensor is shorter than m, n and k need")
        self._bind_torch_stream()
        self._check(self._L.zwg_linear_q8_dev(self._h, self._dev_ptr(x, "x"), m, k, w.q.data_ptr(),
                                              self._dev_ptr(w.scales, "scales"), self._dev_ptr(bias, "bias"), n,
                                              self._dev_ptr(out, "out")))

    def linear_q8w_dev(self, x, m: int, w: "Q8Resident", bias, out) -> None:
        """out[m][w.n] = x[m][w.k] . W^T (+ bias) over resident packed int8 weights: CUDA float32 tensors
        (out may be a raw device address, e.g. a KVCache's rows)."""
        if not isinstance(w, Q8Resident):
            raise ZwgError("w must be a Q8Resident (Q8.resident)")
        if x.numel() < m * w.k or (not isinstance(out, int) and out.numel() < m * w.n) or (
                bias is not None and bias.numel() < w.n):
            raise ZwgError("a tensor is shorter than m, n and k need")
        self._bind_torch_stream()
        self._check(self._L.zwg_linear_q8w_dev(self._h, self._dev_ptr(x, "x"), m, w.handle,
                                               self._dev_ptr(bias, "bias"), self._dev_ptr(out, "out")))

    def linear_q8w_group_dev(self, x, m: int, ws, biases, outs) -> None:
        """outs[j][m][ws[j].n] = x[m][k] . ws[j]^T (+ biases[j]) for up to four resident weight sets
        sharing k, in one x split, stream launch and split sum (zwg_linear_q8w_group_dev)."""
        n_w = len(ws)
        if not 1 <= n_w <= 4 or len(outs) != n_w or (biases is not None and len(biases) != n_w):
            raise ZwgError("one to four weight sets, with as many outputs (and biases)")
        for w, out in zip(ws, outs):
            if not isinstance(w, Q8Resident):
                raise ZwgError("weights must be Q8Resident (Q8.resident)")
            if x.numel() < m * w.k or out.numel() < m * w.n:
                raise ZwgError("a tensor is shorter than m, n and k need")
        bias_list = list(biases) if biases is not None else [None] * n_w
        for w, b in zip(ws, bias_list):
            if b is not None and b.numel() < w.n:
                raise ZwgError("a bias is shorter than n")
        self._bind_torch_stream()
        wa = (ctypes.c_void_p * n_w)(*[w.handle for w in ws])
        ba = (_lib._fp * n_w)(*[self._dev_ptr(b, "bias") for b in bias_list])
        oa = (_lib._fp * n_w)(*[self._dev_ptr(o, "out") for o in outs])
        self._check(self._L.zwg_linear_q8w_group_dev(self._h, self._dev_ptr(x, "x"), m, n_w, wa, ba, oa))

    def linear_q8w_qkv_kv_dev(self, x, m: int, ws, biases, q_out, kv: "KVCache", layer: int, seq0: int,
                              pos_dev) -> None:
        """A decode step's q/k/v projections (resident weights ws = (q, k, v)) with the cache append
        fused into their store: q (rotated when the cache has rotary tables) to q_out, k and v into
        kv's rows of sequences seq0 .. seq0 + m - 1 at the positions of pos_dev (a CUDA int32
        tensor of m entries) -- zwg_linear_q8w_qkv_kv_dev."""
        import torch

        if len(ws) != 3 or (biases is not None and len(biases) != 3):
            raise ZwgError("three weight sets (q, k, v), and three biases or None")
        for w in ws:
            if not isinstance(w, Q8Resident):
                raise ZwgError("weights must be Q8Resident (Q8.resident)")
        if x.numel() < m * ws[0].k or q_out.numel() < m * ws[0].n:
            raise ZwgError("a tensor is shorter than m, n and k need")
        if not pos_dev.is_cuda or pos_dev.dtype != torch.int32 or pos_dev.numel() < m:
            raise ZwgError("pos_dev must be a CUDA int32 tensor with m entries")
        bias_list = list(biases) if biases is not None else [None] * 3
        for w, b in zip(ws, bias_list):
            if b is not None and b.numel() < w.n:
                raise ZwgError("a bias is shorter than n")
        self._bind_torch_stream()
        wa = (ctypes.c_void_p * 3)(*[w.handle for w in ws])
        ba = (_lib._fp * 3)(*[self._dev_ptr(b, "bias") for b in bias_list])
        self._check(self._L.zwg_linear_q8w_qkv_kv_dev(self._h, self._dev_ptr(x, "x"), m, wa, ba,
                                                      self._dev_ptr(q_out, "q_out"), kv._h, layer, seq0,
                                                      pos_dev.data_ptr()))

    def linear_epi_dev(self, x, m: int, k: int, w, bias, n: int, out, epilogue: int, out_stride: int = 0) -> None:
        """linear_dev with an epilogue (_lib.EPI_NONE / EPI_GELU / EPI_ADD) and an output row stride."""
        import torch

        if not isinstance(w, torch.Tensor) or not w.is_cuda or w.dtype != torch.float16:
            raise ZwgError("w must be a CUDA float16 tensor")
        ld = out_stride or n
        if x.numel() < m * k or w.numel() < n * k or (m and out.numel() < (m - 1) * ld + n) or (
                bias is not None and bias.numel() < n):
            raise ZwgError("a tensor is shorter than m, n and k need")
        self._bind_torch_stream()
        self._check(self._L.zwg_linear_epi_dev(self._h, self._dev_ptr(x, "x"), m, k, w.data_ptr(), _lib.W_F16,
                                               self._dev_ptr(bias, "bias"), n, self._dev_ptr(out, "out"), out_stride,
                                               epilogue))

    def linear_q8w_epi_dev(self, x, m: int, w: "Q8Resident", bias, out, epilogue: int) -> None:
        """linear_q8w_dev with an epilogue (_lib.EPI_NONE / EPI_GELU / EPI_ADD)."""
        if not isinstance(w, Q8Resident):
            raise ZwgError("w must be a Q8Resident (Q8.resident)")
        if x.numel() < m * w.k or out.numel() < m * w.n or (bias is not None and bias.numel() < w.n):
            raise ZwgError("a tensor is shorter than m, n and k need")
        self._bind_torch_stream()
        self._check(self._L.zwg_linear_q8w_epi_dev(self._h, self._dev_ptr(x, "x"), m, w.handle,
                                                   self._dev_ptr(bias, "bias"), self._dev_ptr(out, "out"), epilogue))

    def layer_norm_dev(self, x, m: int, n: int, w, b, eps: float, out) -> None:
        """ops.layerNormEps (src/ops.zig:388-395) on CUDA float32 tensors."""
        if x.numel() < m * n or out.numel() < m * n or w.numel() < n or b.numel() < n:
            raise ZwgError("a tensor is shorter than m and n need")
        self._bind_torch_stream()
        self._check(self._L.zwg_layer_norm_dev(self._h, self._dev_ptr(x, "x"), m, n, self._dev_ptr(w, "w"),
                                               self._dev_ptr(b, "b"), eps, self._dev_ptr(out, "out")))

    def rms_norm_dev(self, x, m: int, n: int, w, eps: float, out) -> None:
        """ops.rmsNorm (src/ops.zig:409-427) on CUDA float32 tensors."""
        if x.numel() < m * n or out.numel() < m * n or w.numel() < n:
            raise ZwgError("a tensor is shorter than m and n need")
        self._bind_torch_stream()
        self._check(self._L.zwg_rms_norm_dev(self._h, self._dev_ptr(x, "x"), m, n, self._dev_ptr(w, "w"), eps,
                                             self._dev_ptr(out, "out")))

    def silu_mul_dev(self, gate, up) -> None:
        """ops.siluMul (src/ops.zig:435-439): gate = gate / (1 + e^-gate) * up, CUDA float32 tensors."""
        if up.numel() < gate.numel():
            raise ZwgError("up is shorter than gate")
        self._bind_torch_stream()
        self._check(self._L.zwg_silu_mul_dev(self._h, self._dev_ptr(gate, "gate"), self._dev_ptr(up, "up"),
                                             gate.numel()))

    def gelu_dev(self, x) -> None:
        """ops.gelu (src/ops.zig:335-340) in place on a CUDA float32 tensor."""
        self._bind_torch_stream()
        self._check(self._L.zwg_gelu_dev(self._h, self._dev_ptr(x, "x"), x.numel()))

    def add_dev(self, x, y) -> None:
        """ops.add: x += y, CUDA float32 tensors of one size."""
        if y.numel() != x.numel():
            raise ZwgError("x and y differ in size")
        self._bind_torch_stream()
        self._check(self._L.zwg_add_dev(self._h, self._dev_ptr(x, "x"), self._dev_ptr(y, "y"), x.numel()))

    def encoder_layer_dev(self, x, n_windows: int, n_ctx: int, n_state: int, n_head: int, w: dict, scratch) -> None:
        """One Whisper encoder layer (src/encoder.zig:164-175) over n_windows windows, x [n_windows][n_ctx]
        [n_state] updated in place.  w maps the zwg_enc_layer field names to CUDA tensors (f16 matrices,
        f32 norms and biases); scratch holds encoder_layer_scratch(n_windows * n_ctx, n_state) floats."""
        need = int(self._L.zwg_encoder_layer_scratch(n_windows * n_ctx, n_state))
        if scratch.numel() < need or x.numel() < n_windows * n_ctx * n_state:
            raise ZwgError(f"x or scratch too small (scratch needs {need} floats)")
        ptrs = {}
        for name, _ in _lib.EncLayerC._fields_:  # every field is required (k has no bias field)
            t = w.get(name)
            if t is None or not t.is_cuda or not t.is_contiguous():
                raise ZwgError(f"encoder-layer tensor {name} must be a contiguous CUDA tensor")
            ptrs[name] = t.data_ptr()
        c = _lib.EncLayerC(**ptrs)
        self._bind_torch_stream()
        self._check(self._L.zwg_encoder_layer_dev(self._h, self._dev_ptr(x, "x"), n_windows, n_ctx, n_state, n_head,
                                                  ctypes_byref(c), self._dev_ptr(scratch, "scratch")))

    def attention_dev(self, q, k, v, sh: AttnShape, out) -> None:
        self._bind_torch_stream()
        c = sh.to_c()
        self._check(self._L.zwg_attention_dev(self._h, self._dev_ptr(q, "q"), self._dev_ptr(k, "k"),
                                              self._dev_ptr(v, "v"), ctypes.byref(c), self._dev_ptr(out, "out")))

    def attention_batch_dev(self, q, k, v, sh: AttnShape, out, n_batch: int, q_bstride: int, k_bstride: int,
                            v_bstride: int, out_bstride: int, n_kv_dev=None) -> None:
        """A batch of n_batch problems at fixed strides (floats); n_kv_dev: int32 CUDA tensor or None."""
        import torch

        self._bind_torch_stream()
        nkv = 0
        if n_kv_dev is not None:
            if not n_kv_dev.is_cuda or n_kv_dev.dtype != torch.int32 or n_kv_dev.numel() < n_batch:
                raise ZwgError("n_kv_dev must be a CUDA int32 tensor with n_batch entries")
            nkv = n_kv_dev.data_ptr()
        c = sh.to_c()
        b = _lib.BatchC(n_batch, q_bstride, k_bstride, v_bstride, out_bstride, nkv)
        self._check(self._L.zwg_attention_batch_dev(self._h, self._dev_ptr(q, "q"), self._dev_ptr(k, "k"),
                                                    self._dev_ptr(v, "v"), ctypes.byref(c), ctypes.byref(b),
                                                    self._dev_ptr(out, "out")))


def attention_batch_noalloc(q, k, v, sh: AttnShape, out, n_batch: int = 1, q_bstride: int = 0, k_bstride: int = 0,
                            v_bstride: int = 0, out_bstride: int = 0, n_kv_dev=None, dense_math: int = 0,
                            stream=None) -> None:
    """zwg_attention_batch_noalloc: a batch of problems on CUDA float32 tensors with no context and
    no device allocation (split partials in the library's static scratch, ZWG_NOALLOC_SCRATCH_BYTES
    per GPU), on the current device and `stream` (a torch stream; None: torch's current stream).
    Same plan and results as Context.attention_batch_dev on a context with the default workspace;
    calls on one GPU that overlap in time race on the shared scratch."""
    import torch

    nkv = 0
    if n_kv_dev is not None:
        if not n_kv_dev.is_cuda or n_kv_dev.dtype != torch.int32 or n_kv_dev.numel() < n_batch:
            raise ZwgError("n_kv_dev must be a CUDA int32 tensor with n_batch entries")
        nkv = n_kv_dev.data_ptr()
    s = stream if stream is not None else torch.cuda.current_stream()
    c = sh.to_c()
    b = _lib.BatchC(n_batch, q_bstride, k_bstride, v_bstride, out_bstride, nkv)
    rc = _lib.lib().zwg_attention_batch_noalloc(Context._dev_ptr(q, "q"), Context._dev_ptr(k, "k"),
                                                Context._dev_ptr(v, "v"), ctypes.byref(c), ctypes.byref(b),
                                                Context._dev_ptr(out, "out"), dense_math, s.cuda_stream)
    if rc != _lib.ZWG_OK:
        raise ZwgError(_lib.last_error(None))


class KVCache:
    """Device-resident KV caches of one context (zwg_kv_*): per (layer, sequence), in the Whisper
    decoder's row-major layout (layout=KV_ROW) or Qwen2's transposed-key layout (layout=KV_KT),
    with NeoX rotary positions applied on append when rope_base > 0."""

    def __init__(self, ctx: Context, n_layer: int, n_seq: int, n_ctx: int, n_head_kv: int, d: int,
                 layout: int = _lib.KV_ROW, rope_base: float = 0.0):
        self.ctx = ctx
        self._L = ctx._L
        self.desc = _lib.KVDescC(n_layer, n_seq, n_ctx, n_head_kv, d, layout, 0, rope_base)
        h = ctypes.c_void_p()
        rc = self._L.zwg_kv_create(ctx.handle, ctypes.byref(self.desc), ctypes.byref(h))
        if rc != _lib.ZWG_OK:
            raise ZwgError(_lib.last_error(ctx.handle))
        self._h = h
        self.n_layer, self.n_seq, self.n_ctx, self.n_head_kv, self.d = n_layer, n_seq, n_ctx, n_head_kv, d
        self.layout = layout
        self.kvw = n_head_kv * d
        self.info = _lib.KVInfoC()
        ctx._check(self._L.zwg_kv_get_info(self._h, ctypes.byref(self.info)))
        ctx._adopt(self)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._L.zwg_kv_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def ptrs(self, layer: int, seq: int = 0) -> tuple[int, int]:
        """Device addresses of (layer, seq)'s K and V caches."""
        off = 4 * (layer * self.info.layer_stride + seq * self.info.seq_stride)
        return self.info.k + off, self.info.v + off

    def append(self, layer: int, seq: int, pos: int, k_rows, v_rows, q=None, n_head: int = 0, q_stride: int = 0) -> None:
        """Append rows at pos.. of (layer, seq): CUDA float32 tensors (asynchronous, torch's current
        stream) or float32 numpy arrays (staged, synchronous; q is rotated in place either way)."""
        if isinstance(k_rows, np.ndarray):
            for name, a in (("k_rows", k_rows), ("v_rows", v_rows), ("q", q)):
                if a is not None and (a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]):
                    raise ZwgError(f"{name} must be a contiguous float32 array")
            n = k_rows.size // self.kvw
            self.ctx._check(self._L.zwg_kv_append(self._h, layer, seq, pos, n, k_rows.ctypes.data, v_rows.ctypes.data,
                                                  q.ctypes.data if q is not None else None, n_head, q_stride,
                                                  _lib.ROWS_ON_HOST))
            return
        self.ctx._bind_torch_stream()
        n = k_rows.numel() // self.kvw
        self.ctx._check(self._L.zwg_kv_append(self._h, layer, seq, pos, n, Context._dev_ptr(k_rows, "k_rows"),
                                              Context._dev_ptr(v_rows, "v_rows"), Context._dev_ptr(q, "q"), n_head,
                                              q_stride, 0))

    def append_batch(self, layer: int, seq0: int, pos_dev, k_rows, v_rows, q=None, n_head: int = 0,
                     q_stride: int = 0) -> None:
        """One row per sequence seq0.. at the positions in pos_dev (CUDA int32 tensor)."""
        import torch

        if not pos_dev.is_cuda or pos_dev.dtype != torch.int32:
            raise ZwgError("pos_dev must be a CUDA int32 tensor")
        self.ctx._bind_torch_stream()
        self.ctx._check(self._L.zwg_kv_append_batch(self._h, layer, seq0, pos_dev.numel(), pos_dev.data_ptr(),
                                                    Context._dev_ptr(k_rows, "k_rows"), Context._dev_ptr(v_rows, "v_rows"),
                                                    Context._dev_ptr(q, "q"), n_head, q_stride))

    def read(self, layer: int, seq: int = 0) -> tuple[np.ndarray, np.ndarray]:
        """(K, V) of (layer, seq) on the host, in the cache's layout (synchronous)."""
        k = np.empty(self.n_ctx * self.kvw, np.float32)
        v = np.empty(self.n_ctx * self.kvw, np.float32)
        self.ctx._check(self._L.zwg_kv_read(self._h, layer, seq, k.ctypes.data, v.ctypes.data))
        return k, v


class Decoder:
    """The Whisper text decoder on the device (zwg_decoder_*), src/decoder.zig's Decoder for n_windows
    windows decoded in lockstep: set_audio is Decoder.setAudio (src/decoder.zig:151-159) for a range
    of windows, step is Decoder.forward (src/decoder.zig:165-205) with one token per window.

    layers: one dict per layer mapping the zwg_dec_layer field names (_lib.DEC_LAYER_FIELDS) to a
    Q8 (the matrices) or a float32 array / CUDA tensor (norms, biases; a bias may be None); te: Q8
    [n_vocab][n_state]; pe [n_text_ctx][n_state], ln_w, ln_b [n_state].  The weights are made
    resident and the self and cross caches allocated here; close() frees them."""

    def __init__(self, ctx: Context, te: "Q8", pe, ln_w, ln_b, layers, n_head: int, n_text_ctx: int,
                 n_audio_ctx: int, n_windows: int):
        import torch

        self.ctx = ctx
        self._L = ctx._L
        self.n_vocab, self.n_state, self.n_head, self.n_layer = te.n, te.k, n_head, len(layers)
        self.n_text_ctx, self.n_audio_ctx, self.n_windows = n_text_ctx, n_audio_ctx, n_windows
        self._owned = []  # residents and caches, closed in reverse
        self._keep = []   # device tensors the C structs point at

        def vec(a):
            if a is None:
                return None
            t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a, np.float32))
            t = t.to(device=f"cuda:{ctx.device}", dtype=torch.float32).contiguous()
            self._keep.append(t)
            return t.data_ptr()

        def res(w):
            r = w.resident(ctx)
            self._owned.append(r)
            return r.handle

        d = self.n_state // n_head
        self.te = te.resident(ctx)
        self._owned.append(self.te)
        c_layers = (_lib.DecLayerC * self.n_layer)()
        # per layer, what each field points at: a Q8Resident, a CUDA tensor or None
        self.layer_refs = []
        for li, lw in enumerate(layers):
            vals, refs = {}, {}
            for name in _lib.DEC_LAYER_FIELDS:
                v = lw.get(name)
                vals[name] = res(v) if isinstance(v, Q8) else vec(v)
                refs[name] = (self._owned[-1] if isinstance(v, Q8) else self._keep[-1]) if v is not None else None
            c_layers[li] = _lib.DecLayerC(**vals)
            self.layer_refs.append(refs)
        self.self_kv = KVCache(ctx, self.n_layer, n_windows, n_text_ctx, n_head, d)
        self.cross_kv = KVCache(ctx, self.n_layer, n_windows, n_audio_ctx, n_head, d)
        self._owned += [self.self_kv, self.cross_kv]
        self._layers = c_layers
        pe_p, lnw_p, lnb_p = vec(pe), vec(ln_w), vec(ln_b)
        self.pe, self.ln_w, self.ln_b = self._keep[-3:]
        self.c = _lib.DecoderC(self.n_vocab, self.n_state, n_head, self.n_layer, self.te.handle, pe_p, lnw_p, lnb_p,
                               c_layers, self.self_kv._h.value, self.cross_kv._h.value)
        self.scratch = torch.empty(int(self._L.zwg_decoder_scratch(64, self.n_state)), device=f"cuda:{ctx.device}")

    def set_audio(self, enc, n_windows: int, seq0: int = 0) -> None:
        """Cross K/V of windows seq0 .. seq0 + n_windows - 1 from the encoder output enc
        [n_windows][n_audio_ctx][n_state] (CUDA float32)."""
        if enc.numel() < n_windows * self.n_audio_ctx * self.n_state:
            raise ZwgError("enc is shorter than n_windows x n_audio_ctx x n_state")
        self.ctx._bind_torch_stream()
        self.ctx._check(self._L.zwg_decoder_set_audio_dev(self.ctx.handle, ctypes_byref(self.c),
                                                          Context._dev_ptr(enc, "enc"), n_windows, seq0))

    def step(self, tokens, pos, logits, seq0: int = 0) -> None:
        """One token per window for windows seq0 .. seq0 + m - 1 (tokens, pos: CUDA int32 tensors of m
        entries, pos the windows' n_past); logits [m][n_vocab] (CUDA float32) written."""
        import torch

        m = tokens.numel()
        for name, t in (("tokens", tokens), ("pos", pos)):
            if not t.is_cuda or t.dtype != torch.int32 or t.numel() != m:
                raise ZwgError(f"{name} must be a CUDA int32 tensor of m entries")
        if logits.numel() < m * self.n_vocab:
            raise ZwgError("logits is shorter than m x n_vocab")
        self.ctx._bind_torch_stream()
        self.ctx._check(self._L.zwg_decoder_step_dev(self.ctx.handle, ctypes_byref(self.c), tokens.data_ptr(),
                                                     pos.data_ptr(), m, seq0, Context._dev_ptr(logits, "logits"),
                                                     Context._dev_ptr(self.scratch, "scratch")))

    def close(self) -> None:
        for o in reversed(self._owned):
            o.close()
        self._owned = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class LLM:
    """Qwen2's decode step on the device (zwg_llm_step_dev): src/llm.zig's Model.forward
    (src/llm.zig:169-216) for n_seq sequences decoded in lockstep, one token per sequence per step.

    layers: one dict per layer mapping the zwg_llm_layer field names (_lib.LLM_LAYER_FIELDS) to a
    Q8 (the matrices) or a float32 array / CUDA tensor (norms, biases; a bias may be None); embd:
    Q8 [n_vocab][n_embd]; output: Q8 or None (tied to embd); output_norm [n_embd].  The weights are
    made resident and the cache (transposed keys, rotary base rope_base) allocated here; close()
    frees them."""

    def __init__(self, ctx: Context, embd: "Q8", output, output_norm, layers, n_head: int, n_head_kv: int,
                 n_ff: int, n_ctx: int, n_seq: int, rope_base: float = 1e6, eps: float = 1e-6):
        import torch

        self.ctx = ctx
        self._L = ctx._L
        self.n_vocab, self.n_embd, self.n_head, self.n_head_kv = embd.n, embd.k, n_head, n_head_kv
        self.n_ff, self.n_layer, self.n_ctx, self.n_seq, self.eps = n_ff, len(layers), n_ctx, n_seq, eps
        self._owned, self._keep = [], []

        def vec(a):
            if a is None:
                return None
            t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a, np.float32))
            t = t.to(device=f"cuda:{ctx.device}", dtype=torch.float32).contiguous()
            self._keep.append(t)
            return t.data_ptr()

        def res(w):
            r = w.resident(ctx)
            self._owned.append(r)
            return r.handle

        self.embd = embd.resident(ctx)
        self._owned.append(self.embd)
        self.output = self.embd if output is None else output.resident(ctx)
        if output is not None:
            self._owned.append(self.output)
        c_layers = (_lib.LlmLayerC * self.n_layer)()
        self.layer_refs = []
        for li, lw in enumerate(layers):
            vals, refs = {}, {}
            for name in _lib.LLM_LAYER_FIELDS:
                v = lw.get(name)
                vals[name] = res(v) if isinstance(v, Q8) else vec(v)
                refs[name] = (self._owned[-1] if isinstance(v, Q8) else self._keep[-1]) if v is not None else None
            c_layers[li] = _lib.LlmLayerC(**vals)
            self.layer_refs.append(refs)
        self.kv = KVCache(ctx, self.n_layer, n_seq, n_ctx, n_head_kv, self.n_embd // n_head, _lib.KV_KT, rope_base)
        self._owned.append(self.kv)
        self._layers = c_layers
        on_p = vec(output_norm)
        self.output_norm = self._keep[-1]
        self.c = _lib.LlmC(self.n_vocab, self.n_embd, n_head, n_head_kv, n_ff, self.n_layer, eps, 0, self.embd.handle,
                           self.output.handle, on_p, c_layers, self.kv._h.value)
        self.scratch = torch.empty(int(self._L.zwg_llm_scratch(64, self.n_embd, n_ff)), device=f"cuda:{ctx.device}")

    def step(self, tokens, pos, logits, seq0: int = 0) -> None:
        """One token per sequence for sequences seq0 .. seq0 + m - 1 (tokens, pos: CUDA int32 tensors
        of m entries, pos the sequences' n_past); logits [m][n_vocab] (CUDA float32) written."""
        import torch

        m = tokens.numel()
        for name, t in (("tokens", tokens), ("pos", pos)):
            if not t.is_cuda or t.dtype != torch.int32 or t.numel() != m:
                raise ZwgError(f"{name} must be a CUDA int32 tensor of m entries")
        if logits.numel() < m * self.n_vocab:
            raise ZwgError("logits is shorter than m x n_vocab")
        self.ctx._bind_torch_stream()
        self.ctx._check(self._L.zwg_llm_step_dev(self.ctx.handle, ctypes_byref(self.c), tokens.data_ptr(),
                                                 pos.data_ptr(), m, seq0, Context._dev_ptr(logits, "logits"),
                                                 Context._dev_ptr(self.scratch, "scratch")))

    def forward(self, tokens, pos0: int, logits, seq: int = 0) -> None:
        """Model.forward over the n tokens of `tokens` (a CUDA int32 tensor) of sequence seq at
        positions pos0 .. pos0 + n - 1 (the reference's prompt batch); logits [n_vocab] (CUDA
        float32) get the last token's (zwg_llm_forward_dev)."""
        import torch

        n = tokens.numel()
        if not tokens.is_cuda or tokens.dtype != torch.int32:
            raise ZwgError("tokens must be a CUDA int32 tensor")
        if logits.numel() < self.n_vocab:
            raise ZwgError("logits is shorter than n_vocab")
        need = int(self._L.zwg_llm_forward_scratch(n, self.n_embd, self.n_ff))
        if getattr(self, "_fwd_scratch", None) is None or self._fwd_scratch.numel() < need:
            self._fwd_scratch = torch.empty(max(need, 4), device=f"cuda:{self.ctx.device}")
        self.ctx._bind_torch_stream()
        self.ctx._check(self._L.zwg_llm_forward_dev(self.ctx.handle, ctypes_byref(self.c), tokens.data_ptr(), n, seq,
                                                    pos0, Context._dev_ptr(logits, "logits"),
                                                    Context._dev_ptr(self._fwd_scratch, "scratch")))

    def close(self) -> None:
        for o in reversed(self._owned):
            o.close()
        self._owned = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


_tls = threading.local()


def ctypes_byref(c):
    import ctypes

    return ctypes.byref(c)


def encoder_layer_scratch(n_rows: int, n_state: int) -> int:
    """Floats of scratch zwg_encoder_layer_dev needs for n_rows rows (windows x frames)."""
    return int(_lib.lib().zwg_encoder_layer_scratch(n_rows, n_state))


def default_context() -> Context:
    """The calling thread's context on device 0, opened on first use."""
    ctx = getattr(_tls, "ctx", None)
    if ctx is None:
        ctx = Context(0)
        _tls.ctx = ctx
    return ctx


def _as_f32(a, name: str) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype != np.float32:
        raise ZwgError(f"{name} must be float32")
    return np.ascontiguousarray(a).reshape(-1)


def attentionEx(pool, q, k, v, sh: AttnShape, scratch, out) -> None:
    """ops.attentionEx (src/ops.zig:562) on host buffers; `out` (float32, contiguous) is written in place."""
    del pool, scratch
    if not isinstance(out, np.ndarray) or out.dtype != np.float32 or not out.flags["C_CONTIGUOUS"]:
        raise ZwgError("out must be a contiguous float32 numpy array")
    q, k, v = _as_f32(q, "q"), _as_f32(k, "k"), _as_f32(v, "v")
    default_context().attention_ex_host(q, k, v, sh, out.reshape(-1))


Q8_BLOCK = 32  # src/gemm.zig:194


class Q8:
    """gemm.Q8 (src/gemm.zig:196-266): int8 weights q [n][k] and f32 scales [n][k / 32], one per block
    of 32 weights of a row (absmax / 127).  Holds numpy arrays (host) or CUDA tensors (to_device)."""

    def __init__(self, q, scales, n: int, k: int):
        if k % Q8_BLOCK:
            raise ZwgError("k must be a multiple of 32")
        self.q, self.scales, self.n, self.k = q, scales, int(n), int(k)

    def blocks(self) -> int:
        return self.k // Q8_BLOCK

    @classmethod
    def quantize(cls, w, n: int, k: int) -> "Q8":
        """Q8.quantize (src/gemm.zig:209-230) of an [n][k] f16 or f32 matrix: scale = amax / 127 in f32,
        q = clamp(round(v * (127 / amax)), -127, 127) with ties away from zero (Zig's @round)."""
        if k % Q8_BLOCK:
            raise ZwgError("k must be a multiple of 32")
        w = np.asarray(w).reshape(-1)[: n * k].astype(np.float32).reshape(n, k // Q8_BLOCK, Q8_BLOCK)
        amax = np.abs(w).max(axis=2)
        scale = (amax / np.float32(127.0)).astype(np.float32)
        with np.errstate(divide="ignore"):
            inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0)).astype(np.float32)
        r = (w * inv[:, :, None]).astype(np.float32).astype(np.float64)
        r = np.sign(r) * np.floor(np.abs(r) + 0.5)  # exact in f64 for any f32 product
        q = np.clip(r, -127, 127).astype(np.int8).reshape(n, k)
        return cls(q, scale.reshape(n, k // Q8_BLOCK), n, k)

    @classmethod
    def from_q8_0(cls, data: bytes, n: int, k: int) -> "Q8":
        """Q8.fromQ8_0 (src/gemm.zig:232-248): GGUF q8_0 blocks (f16 scale, then 32 int8) to the same
        int8 and f32 scales."""
        if k % Q8_BLOCK:
            raise ZwgError("k must be a multiple of 32")
        nb = k // Q8_BLOCK
        blk = np.frombuffer(data, dtype=np.uint8, count=n * nb * 34).reshape(n * nb, 34)
        scales = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(n, nb)
        q = blk[:, 2:].copy().view(np.int8).reshape(n, k)
        return cls(q, scales, n, k)

    def row(self, i: int) -> np.ndarray:
        """Q8.row (src/gemm.zig:255-263): row i dequantized, f32(q) * scale."""
        q = np.asarray(self.q).reshape(self.n, self.k)[i].astype(np.float32).reshape(-1, Q8_BLOCK)
        return (q * np.asarray(self.scales, np.float32).reshape(self.n, -1)[i][:, None]).reshape(-1)

    def resident(self, ctx: "Context") -> "Q8Resident":
        """These weights uploaded once into HBM in the packed device layout (zwg_q8w_create): the
        GPU form of building the Q8 at load.  From host arrays or CUDA tensors."""
        return Q8Resident(ctx, self)

    def to_device(self, device: int = 0) -> "Q8":
        """The same weights as CUDA tensors (int8 q, float32 scales), for Context.linear_q8_dev."""
        import torch

        q = torch.as_tensor(np.ascontiguousarray(np.asarray(self.q, np.int8).reshape(self.n, self.k)))
        s = torch.as_tensor(np.ascontiguousarray(np.asarray(self.scales, np.float32).reshape(self.n, -1)))
        return Q8(q.to(f"cuda:{device}"), s.to(f"cuda:{device}"), self.n, self.k)


class Q8Resident:
    """Int8 block weights resident in HBM in the packed device layout (zwg_q8w).  Use with
    Context.linear_q8w_dev; close() (or the context manager) frees them, before the context."""

    def __init__(self, ctx: "Context", w: Q8):
        import ctypes

        self.ctx, self.n, self.k = ctx, w.n, w.k
        h = ctypes.c_void_p()
        if isinstance(w.q, np.ndarray):
            q = np.ascontiguousarray(w.q, dtype=np.int8)
            sc = np.ascontiguousarray(w.scales, dtype=np.float32)
            if q.size < w.n * w.k or sc.size < w.n * (w.k // Q8_BLOCK):
                raise ZwgError("q or scales shorter than [n][k] needs")
            rc = ctx._L.zwg_q8w_create(ctx.handle, q.ctypes.data, sc.ctypes.data, w.n, w.k, _lib.Q8W_FROM_HOST,
                                       ctypes.byref(h))
        else:
            import torch

            if not (isinstance(w.q, torch.Tensor) and w.q.is_cuda and w.q.dtype == torch.int8
                    and w.q.is_contiguous() and w.scales.is_contiguous()):
                raise ZwgError("w must hold contiguous host arrays or CUDA int8 / float32 tensors")
            if w.q.numel() < w.n * w.k or w.scales.numel() < w.n * (w.k // Q8_BLOCK):
                raise ZwgError("q or scales shorter than [n][k] needs")
            ctx._bind_torch_stream()
            rc = ctx._L.zwg_q8w_create(ctx.handle, w.q.data_ptr(), Context._dev_ptr(w.scales, "scales"), w.n, w.k, 0,
                                       ctypes.byref(h))
        ctx._check(rc)
        self._h = h.value
        ctx._adopt(self)

    @property
    def handle(self):
        if not self._h:
            raise ZwgError("weights are closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.ctx._L.zwg_q8w_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def linear(pool, x, m: int, k: int, w, b, n: int, out) -> None:
    """ops.linear (src/ops.zig:283-306): out[i][o] = sum_p x[i][p] * w[o][p] (+ b[o]).  w is a float16
    [n][k] array or a Q8 (int8 block weights), as the reference's `anytype`; x f32 [m][k], b f32 [n] or
    None, out f32 [m][n]; host arrays, synchronous."""
    del pool  # the GPU context replaces the thread pool
    x = _as_f32(x, "x")
    if isinstance(w, Q8):
        _linear_q8_host(x, m, k, w, b, n, out)
        return
    w = np.asarray(w)
    if w.dtype != np.float16 or not w.flags["C_CONTIGUOUS"]:
        raise ZwgError("w must be a contiguous float16 array")
    bb = None if b is None else _as_f32(b, "b")
    if not isinstance(out, np.ndarray) or out.dtype != np.float32 or not out.flags["C_CONTIGUOUS"]:
        raise ZwgError("out must be a contiguous float32 array")
    if x.size < m * k or w.size < n * k or out.size < m * n or (bb is not None and bb.size < n):
        raise ZwgError("a buffer is shorter than m, n and k need")
    ctx = default_context()
    ctx._check(ctx._L.zwg_linear(ctx.handle, x.ctypes.data, m, k, w.ctypes.data, _lib.W_F16,
                                 None if bb is None else bb.ctypes.data, n, out.ctypes.data))


def _linear_q8_host(x, m: int, k: int, w: Q8, b, n: int, out) -> None:
    q = np.asarray(w.q)
    sc = np.asarray(w.scales)
    if q.dtype != np.int8 or sc.dtype != np.float32 or not q.flags["C_CONTIGUOUS"] or not sc.flags["C_CONTIGUOUS"]:
        raise ZwgError("w must hold contiguous int8 q and float32 scales (host arrays)")
    if w.n != n or w.k != k:
        raise ZwgError(f"w is [{w.n}][{w.k}], the call asks for [{n}][{k}]")
    bb = None if b is None else _as_f32(b, "b")
    if not isinstance(out, np.ndarray) or out.dtype != np.float32 or not out.flags["C_CONTIGUOUS"]:
        raise ZwgError("out must be a contiguous float32 array")
    if x.size < m * k or q.size < n * k or sc.size < n * (k // Q8_BLOCK) or out.size < m * n or (
            bb is not None and bb.size < n):
        raise ZwgError("a buffer is shorter than m, n and k need")
    ctx = default_context()
    ctx._check(ctx._L.zwg_linear_q8(ctx.handle, x.ctypes.data, m, k, q.ctypes.data, sc.ctypes.data,
                                    None if bb is None else bb.ctypes.data, n, out.ctypes.data))


def attention(pool, q, k, v, n_q: int, n_kv: int, n_state: int, n_head: int, causal: bool, scratch, out) -> None:
    """ops.attention (src/ops.zig:593)."""
    if n_head == 0:
        raise ZwgError("n_head must be positive")
    d = n_state // n_head
    attentionEx(pool, q, k, v, AttnShape(n_q, n_kv, n_head, n_head, d, n_state, n_state, n_state, causal), scratch,
                out)
