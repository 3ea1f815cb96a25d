// Device helpers shared by the elementwise kernels (elementwise.hip) and the linear-layer
// epilogues (linear_kernel.hpp, linear_q8_kernel.hpp), and the host entry of the layer norm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct zwg_ctx;

namespace zwg_ew {

// ggml's GELU, tanh form (src/ops.zig:312-327): u = c (x + 0.044715 x^3), c = sqrt(2/pi),
// tanh(u) = 1 - 2 / (1 + e^(2u)), gelu = 0.5 x (1 + tanh(u)).  Rounded step by step in the
// reference's order (k x x x left to right), with no fused multiply-adds.
__device__ __forceinline__ float gelu(float x) {
#pragma clang fp contract(off)
    const float c = 0.7978845608028654f;
    const float k = 0.044715f;
    const float u = c * (x + k * x * x * x);
    const float t = 1.0f - 2.0f / (1.0f + expf(2.0f * u));
    return 0.5f * x * (1.0f + t);
}

// Linear-layer epilogues (include/zw_gpu.h ZWG_EPI_*): the value v = x . w + b of out[i][o] is
// stored as v, gelu(v), or out[i][o] + v (ops.linear followed by ops.gelu or ops.add).
constexpr uint32_t kEpiNone = 0, kEpiGelu = 1, kEpiAdd = 2;

__device__ __forceinline__ void epilogue_store(float *p, float v, uint32_t epi) {
    if (epi == kEpiGelu) v = gelu(v);
    else if (epi == kEpiAdd) {
#pragma clang fp contract(off)
        v = *p + v;
    }
    *p = v;
}

} // namespace zwg_ew

namespace zwg_host {
int layer_norm(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, const float *b, float eps,
               float *out);
} // namespace zwg_host
