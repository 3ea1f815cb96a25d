"""zwhisper_amd: zwhisper's attention hot path (src/ops.zig:464-605) on AMD MI355X (gfx950).

The compute is libzwgpu.so (HIP, built by ``python -m zwhisper_amd.build``) behind the C ABI in
include/zw_gpu.h; ``zwhisper_amd.ops`` mirrors the reference's ``ops`` interface on top of it, and
``KVCache`` keeps the decoder and LLM caches in HBM (the cache writes of src/decoder.zig:182-183
and src/llm.zig:182-190), ``Decoder`` runs the Whisper text decoder's token steps on the device
(src/decoder.zig:151-205) and ``LLM`` Qwen2's (src/llm.zig:169-216).
"""
from ._lib import DENSE_X3, DENSE_FP32, KV_KT, KV_ROW, ZwgError
from .ops import (AttnShape, Context, Decoder, KVCache, LLM, V, attention, attentionEx, attentionScratch, attentionScratchEx,
                  attentionScratchKT, check_shape, default_context, linear, plan, q_block, Q8, Q8Resident)

__all__ = [
    "AttnShape", "Context", "Decoder", "LLM", "DENSE_X3", "DENSE_FP32", "KVCache", "KV_KT", "KV_ROW", "V", "ZwgError", "attention", "attentionEx",
    "attentionScratch", "attentionScratchEx", "attentionScratchKT", "check_shape", "default_context", "linear", "plan",
    "Q8", "Q8Resident", "q_block",
]
