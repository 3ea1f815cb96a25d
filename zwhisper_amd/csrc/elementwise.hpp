// Device helpers shared by the elementwise kernels (elementwise.hip) and the linear-layer
// epilogues (linear_kernel.hpp, linear_q8_kernel.hpp), and the host entry of the layer norm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct zwg_ctx;

namespace zwg_ew {

// ggml's GELU, tanh form (src/ops.zig:312-327): u = c (x + 0.044715 x^3), c = sqrt(2/pi),
// tanh(u) = 1 - 2 / (1 + e^(2u)), gelu = 0.5 x (1 + tanh(u)).  Rounded step by step in the
// reference's order (k x x x left to right), with no fused multiply-adds.  e^(2u) is 2^(2u log2 e)
// on v_exp_f32 and 2 / (1 + e) is 2 rcp(1 + e) on v_rcp_f32, each within about 1 ulp: the
// rounding of 2u log2 e moves e by at most 2^-24 |2u| relatively, which changes tanh by at most
// 2^-24 where it is not saturated (2e / (1 + e)^2 |2u| <= 1), far below the f32 sums feeding it.
// Large |u| saturate exactly: e = inf gives t = 1, e = 0 gives t = -1.
__device__ __forceinline__ float gelu(float x) {
#pragma clang fp contract(off)
    const float c = 0.7978845608028654f;
    const float k = 0.044715f;
    const float u = c * (x + k * x * x * x);
    const float e = __builtin_amdgcn_exp2f(2.0f * u * 1.4426950408889634f);
    const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
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

typedef float ew_f32x4 __attribute__((ext_vector_type(4)));

// float4 per lane a row held in registers may take: rows up to 64 * 4 * 8 = 2048 floats
constexpr int kNormRegs = 8;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ops.layerNormEps (src/ops.zig:355-381) of one row of n = 4 n4 floats held by one wave: lane l
// holds float4 c = l + 64 i in v[i] (R >= ceil(n4 / 64); zeros past n4).  mean = sum / n, var =
// sum((x - mean)^2) / n (the reference's two passes), inv = 1 / sqrt(var + eps), out = fma((x -
// mean) * inv, w, b).  The sums are reduced across the wave by butterfly, so their rounding order
// differs from the reference's 16-lane vector order (a few f32 ulps).  Every kernel that normalises
// a row goes through this function, so a fused norm equals the separate one bit for bit.
// copy: nullptr, or a second destination of the output float4s (same index as in orow).
template <int R>
__device__ __forceinline__ void layer_norm_regs(const ew_f32x4 (&v)[R], int lane, int n4, const float *w,
                                                const float *b, float eps, float *orow, ew_f32x4 *copy = nullptr) {
    const float fn = (float)(4 * n4);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < R; ++i) s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
    const float mean = wave_sum(s) / fn;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        if (c < n4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = v[i][e] - mean;
                q = __builtin_fmaf(d, d, q);
            }
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / fn + eps);
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        if (c < n4) {
            const ew_f32x4 wv = reinterpret_cast<const ew_f32x4 *>(w)[c];
            const ew_f32x4 bv = reinterpret_cast<const ew_f32x4 *>(b)[c];
            ew_f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf((v[i][e] - mean) * inv, wv[e], bv[e]);
            reinterpret_cast<ew_f32x4 *>(orow)[c] = o;
            if (copy) copy[c] = o;
        }
    }
}

// ops.rmsNorm (src/ops.zig:409-427) of one row held by one wave as for layer_norm_regs: ss = sum of
// x^2 (each lane's fmas, then a butterfly sum across the wave), inv = 1 / sqrt(ss / n + eps), out
// = x * inv * w, multiplied left to right.  Every kernel that RMS-normalises a row goes through
// this function.
template <int R>
__device__ __forceinline__ void rms_norm_regs(const ew_f32x4 (&v)[R], int lane, int n4, const float *w, float eps,
                                              float *orow, ew_f32x4 *copy = nullptr) {
    const float fn = (float)(4 * n4);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        if (c < n4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) q = __builtin_fmaf(v[i][e], v[i][e], q);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / fn + eps);
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        if (c < n4) {
            const ew_f32x4 wv = reinterpret_cast<const ew_f32x4 *>(w)[c];
            ew_f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
                const float r = v[i][e] * inv;
                o[e] = r * wv[e];
            }
            reinterpret_cast<ew_f32x4 *>(orow)[c] = o;
            if (copy) copy[c] = o;
        }
    }
}

// The row norms of the fused kernels: layer norm (w, b) or RMS norm (w; b unused)
constexpr int kNormLayer = 0, kNormRms = 1;
template <int KIND, int R>
__device__ __forceinline__ void norm_regs(const ew_f32x4 (&v)[R], int lane, int n4, const float *w, const float *b,
                                          float eps, float *orow, ew_f32x4 *copy = nullptr) {
    if constexpr (KIND == kNormRms) rms_norm_regs<R>(v, lane, n4, w, eps, orow, copy);
    else layer_norm_regs<R>(v, lane, n4, w, b, eps, orow, copy);
}

// ops.siluMul's element (src/ops.zig:429-439): gate / (1 + e^-gate) * up, rounded step by step in
// that order (no contraction); e^x is the device's expf.
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
    const float s = g / (1.0f + expf(-g));
    return s * u;
}

} // namespace zwg_ew

namespace zwg_host {
int layer_norm(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, const float *b, float eps,
               float *out);
int rms_norm(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, float eps, float *out);
} // namespace zwg_host
