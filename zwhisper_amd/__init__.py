"""zwhisper_amd: zwhisper's attention hot path (src/ops.zig:464-605) on AMD MI355X (gfx950).

The compute is libzwgpu.so (HIP, built by ``python -m zwhisper_amd.build``) behind the C ABI in
include/zw_gpu.h; ``zwhisper_amd.ops`` mirrors the reference's ``ops`` interface on top of it.
"""
from ._lib import ZwgError
from .ops import (AttnShape, Context, V, attention, attentionEx, attentionScratch, attentionScratchEx,
                  attentionScratchKT, check_shape, default_context, plan, q_block)

__all__ = [
    "AttnShape", "Context", "V", "ZwgError", "attention", "attentionEx", "attentionScratch", "attentionScratchEx",
    "attentionScratchKT", "check_shape", "default_context", "plan", "q_block",
]
