"""ctypes binding of include/zw_gpu.h (libzwgpu.so, built in-tree by zwhisper_amd/build.py).

Loading fails loudly when the library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libzwgpu.so")
HEADER = os.path.join(ROOT, "include", "zw_gpu.h")

ZWG_OK = 0
ZWG_ERROR = 2

_u64 = ctypes.c_uint64
_fp = ctypes.c_void_p  # device or host float pointers travel as addresses


class ZwgError(RuntimeError):
    """A call into the library returned ZWG_ERROR (the message is zwg_last_error)."""


class ShapeC(ctypes.Structure):
    _fields_ = [
        ("n_q", _u64),
        ("n_kv", _u64),
        ("n_head", _u64),
        ("n_head_kv", _u64),
        ("d", _u64),
        ("q_stride", _u64),
        ("kv_stride", _u64),
        ("out_stride", _u64),
        ("kt_stride", _u64),
        ("causal", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class BatchC(ctypes.Structure):
    _fields_ = [
        ("n_batch", _u64),
        ("q_bstride", _u64),
        ("k_bstride", _u64),
        ("v_bstride", _u64),
        ("out_bstride", _u64),
        ("n_kv_dev", ctypes.c_void_p),
    ]


class LimitsC(ctypes.Structure):
    _fields_ = [("workspace_bytes", _u64), ("dense_math", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("staging_bytes", _u64)]


class PlanC(ctypes.Structure):
    _fields_ = [
        ("kernel", ctypes.c_uint32),
        ("rows_per_unit", ctypes.c_uint32),
        ("chunk_len", _u64),
        ("max_chunks", _u64),
        ("grid_blocks", _u64),
        ("workspace_bytes", _u64),
    ]


class EncLayerC(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "attn_ln_w", "attn_ln_b", "q_w", "q_b", "k_w", "v_w", "v_b", "o_w", "o_b", "mlp_ln_w", "mlp_ln_b", "mlp0_w",
        "mlp0_b", "mlp1_w", "mlp1_b")]


DEC_LAYER_FIELDS = ("attn_ln_w", "attn_ln_b", "q_w", "q_b", "k_w", "v_w", "v_b", "o_w", "o_b", "cross_ln_w",
                    "cross_ln_b", "cq_w", "cq_b", "ck_w", "cv_w", "cv_b", "co_w", "co_b", "mlp_ln_w", "mlp_ln_b",
                    "mlp0_w", "mlp0_b", "mlp1_w", "mlp1_b")


class DecLayerC(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in DEC_LAYER_FIELDS]


class DecoderC(ctypes.Structure):
    _fields_ = [
        ("n_vocab", _u64),
        ("n_state", _u64),
        ("n_head", _u64),
        ("n_layer", _u64),
        ("te", ctypes.c_void_p),
        ("pe", ctypes.c_void_p),
        ("ln_w", ctypes.c_void_p),
        ("ln_b", ctypes.c_void_p),
        ("layers", ctypes.POINTER(DecLayerC)),
        ("self_kv", ctypes.c_void_p),
        ("cross_kv", ctypes.c_void_p),
    ]


LLM_LAYER_FIELDS = ("attn_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "ffn_norm", "w_gate", "w_up", "w_down")


class LlmLayerC(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in LLM_LAYER_FIELDS]


class LlmC(ctypes.Structure):
    _fields_ = [
        ("n_vocab", _u64),
        ("n_embd", _u64),
        ("n_head", _u64),
        ("n_head_kv", _u64),
        ("n_ff", _u64),
        ("n_layer", _u64),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_uint32),
        ("embd", ctypes.c_void_p),
        ("output", ctypes.c_void_p),
        ("output_norm", ctypes.c_void_p),
        ("layers", ctypes.POINTER(LlmLayerC)),
        ("kv", ctypes.c_void_p),
    ]


class KVDescC(ctypes.Structure):
    _fields_ = [
        ("n_layer", _u64),
        ("n_seq", _u64),
        ("n_ctx", _u64),
        ("n_head_kv", _u64),
        ("d", _u64),
        ("layout", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("rope_base", ctypes.c_double),
    ]


class KVInfoC(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("layer_stride", _u64),
        ("seq_stride", _u64),
        ("kv_stride", _u64),
        ("kt_stride", _u64),
    ]


DENSE_X3 = 0
DENSE_FP32 = 1
KV_ROW = 0
KV_KT = 1
W_F16 = 1
W_Q8 = 2
Q8W_FROM_HOST = 1
EPI_NONE = 0
EPI_GELU = 1
EPI_ADD = 2
ROWS_ON_HOST = 1
NOALLOC_SCRATCH_BYTES = 64 << 20  # ZWG_NOALLOC_SCRATCH_BYTES


def declared_symbols() -> list[str]:
    """Every function the C header declares."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(zwg_[a-z_0-9]+)\s*\(", text)))


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `python -m zwhisper_amd.build` (hipcc, gfx950)")
    L = ctypes.CDLL(LIB_PATH)
    c_int, vp = ctypes.c_int, ctypes.c_void_p
    L.zwg_version.restype = c_int
    L.zwg_last_error.restype = ctypes.c_char_p
    L.zwg_last_error.argtypes = [vp]
    L.zwg_open.restype = c_int
    L.zwg_open.argtypes = [c_int, ctypes.POINTER(LimitsC), ctypes.POINTER(vp)]
    L.zwg_close.restype = None
    L.zwg_close.argtypes = [vp]
    L.zwg_set_stream.restype = c_int
    L.zwg_set_stream.argtypes = [vp, vp]
    L.zwg_get_stream.restype = vp
    L.zwg_get_stream.argtypes = [vp]
    L.zwg_sync.restype = c_int
    L.zwg_sync.argtypes = [vp]
    L.zwg_set_dense_math.restype = c_int
    L.zwg_set_dense_math.argtypes = [vp, ctypes.c_uint32]
    L.zwg_attention_ex.restype = c_int
    L.zwg_attention_ex.argtypes = [vp, _fp, _fp, _fp, ctypes.POINTER(ShapeC), _fp]
    L.zwg_attention.restype = c_int
    L.zwg_attention.argtypes = [vp, _fp, _fp, _fp, _u64, _u64, _u64, _u64, c_int, _fp]
    L.zwg_attention_dev.restype = c_int
    L.zwg_attention_dev.argtypes = [vp, _fp, _fp, _fp, ctypes.POINTER(ShapeC), _fp]
    L.zwg_attention_batch_dev.restype = c_int
    L.zwg_attention_batch_dev.argtypes = [vp, _fp, _fp, _fp, ctypes.POINTER(ShapeC), ctypes.POINTER(BatchC), _fp]
    L.zwg_attention_batch_noalloc.restype = c_int
    L.zwg_attention_batch_noalloc.argtypes = [_fp, _fp, _fp, ctypes.POINTER(ShapeC), ctypes.POINTER(BatchC), _fp,
                                              ctypes.c_uint32, vp]
    L.zwg_plan.restype = c_int
    L.zwg_plan.argtypes = [ctypes.POINTER(ShapeC), ctypes.POINTER(BatchC), _u64, ctypes.POINTER(PlanC)]
    L.zwg_check_shape.restype = c_int
    L.zwg_check_shape.argtypes = [ctypes.POINTER(ShapeC), ctypes.c_char_p, ctypes.c_size_t]
    L.zwg_kv_create.restype = c_int
    L.zwg_kv_create.argtypes = [vp, ctypes.POINTER(KVDescC), ctypes.POINTER(vp)]
    L.zwg_kv_destroy.restype = None
    L.zwg_kv_destroy.argtypes = [vp]
    L.zwg_kv_get_info.restype = c_int
    L.zwg_kv_get_info.argtypes = [vp, ctypes.POINTER(KVInfoC)]
    L.zwg_kv_append.restype = c_int
    L.zwg_kv_append.argtypes = [vp, _u64, _u64, _u64, _u64, _fp, _fp, _fp, _u64, _u64, ctypes.c_uint32]
    L.zwg_kv_append_batch.restype = c_int
    L.zwg_kv_append_batch.argtypes = [vp, _u64, _u64, _u64, vp, _fp, _fp, _fp, _u64, _u64]
    L.zwg_kv_read.restype = c_int
    L.zwg_kv_read.argtypes = [vp, _u64, _u64, _fp, _fp]
    for name in ("zwg_linear", "zwg_linear_dev"):
        getattr(L, name).restype = c_int
        getattr(L, name).argtypes = [vp, _fp, _u64, _u64, vp, ctypes.c_uint32, _fp, _u64, _fp]
    L.zwg_q8w_create.restype = c_int
    L.zwg_q8w_create.argtypes = [vp, vp, _fp, _u64, _u64, ctypes.c_uint32, ctypes.POINTER(vp)]
    L.zwg_q8w_destroy.restype = None
    L.zwg_q8w_destroy.argtypes = [vp]
    L.zwg_q8w_shape.restype = c_int
    L.zwg_q8w_shape.argtypes = [vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]
    L.zwg_linear_q8w_dev.restype = c_int
    L.zwg_linear_q8w_dev.argtypes = [vp, _fp, _u64, vp, _fp, _fp]
    L.zwg_linear_q8w_epi_dev.restype = c_int
    L.zwg_linear_q8w_epi_dev.argtypes = [vp, _fp, _u64, vp, _fp, _fp, ctypes.c_uint32]
    L.zwg_linear_q8w_group_dev.restype = c_int
    L.zwg_linear_q8w_group_dev.argtypes = [vp, _fp, _u64, ctypes.c_uint32, ctypes.POINTER(vp), ctypes.POINTER(_fp),
                                           ctypes.POINTER(_fp)]
    L.zwg_linear_q8w_qkv_kv_dev.restype = c_int
    L.zwg_linear_q8w_qkv_kv_dev.argtypes = [vp, _fp, _u64, ctypes.POINTER(vp), ctypes.POINTER(_fp), _fp, vp, _u64,
                                            _u64, vp]
    L.zwg_linear_epi_dev.restype = c_int
    L.zwg_linear_epi_dev.argtypes = [vp, _fp, _u64, _u64, vp, ctypes.c_uint32, _fp, _u64, _fp, _u64, ctypes.c_uint32]
    L.zwg_layer_norm_dev.restype = c_int
    L.zwg_layer_norm_dev.argtypes = [vp, _fp, _u64, _u64, _fp, _fp, ctypes.c_float, _fp]
    L.zwg_gelu_dev.restype = c_int
    L.zwg_gelu_dev.argtypes = [vp, _fp, _u64]
    L.zwg_add_dev.restype = c_int
    L.zwg_add_dev.argtypes = [vp, _fp, _fp, _u64]
    L.zwg_encoder_layer_scratch.restype = _u64
    L.zwg_encoder_layer_scratch.argtypes = [_u64, _u64]
    L.zwg_encoder_layer_dev.restype = c_int
    L.zwg_encoder_layer_dev.argtypes = [vp, _fp, _u64, _u64, _u64, _u64, ctypes.POINTER(EncLayerC), _fp]
    L.zwg_rms_norm_dev.restype = c_int
    L.zwg_rms_norm_dev.argtypes = [vp, _fp, _u64, _u64, _fp, ctypes.c_float, _fp]
    L.zwg_silu_mul_dev.restype = c_int
    L.zwg_silu_mul_dev.argtypes = [vp, _fp, _fp, _u64]
    L.zwg_llm_scratch.restype = _u64
    L.zwg_llm_scratch.argtypes = [_u64, _u64, _u64]
    L.zwg_llm_step_dev.restype = c_int
    L.zwg_llm_step_dev.argtypes = [vp, ctypes.POINTER(LlmC), vp, vp, _u64, _u64, _fp, _fp]
    L.zwg_llm_forward_scratch.restype = _u64
    L.zwg_llm_forward_scratch.argtypes = [_u64, _u64, _u64]
    L.zwg_llm_forward_dev.restype = c_int
    L.zwg_llm_forward_dev.argtypes = [vp, ctypes.POINTER(LlmC), vp, _u64, _u64, _u64, _fp, _fp]
    L.zwg_decoder_set_audio_dev.restype = c_int
    L.zwg_decoder_set_audio_dev.argtypes = [vp, ctypes.POINTER(DecoderC), _fp, _u64, _u64]
    L.zwg_decoder_scratch.restype = _u64
    L.zwg_decoder_scratch.argtypes = [_u64, _u64]
    L.zwg_decoder_step_dev.restype = c_int
    L.zwg_decoder_step_dev.argtypes = [vp, ctypes.POINTER(DecoderC), vp, vp, _u64, _u64, _fp, _fp]
    for name in ("zwg_linear_q8", "zwg_linear_q8_dev"):
        getattr(L, name).restype = c_int
        getattr(L, name).argtypes = [vp, _fp, _u64, _u64, vp, _fp, _fp, _u64, _fp]
    _lib = L
    return L


def last_error(ctx=None) -> str:
    msg = lib().zwg_last_error(ctx)
    return msg.decode() if msg else ""


def check(rc: int, ctx=None) -> None:
    if rc != ZWG_OK:
        raise ZwgError(last_error(ctx))
