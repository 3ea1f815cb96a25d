// Row-wise and elementwise ops around the linear layers and attention (include/zw_gpu.h):
// ops.layerNorm / layerNormEps (src/ops.zig:342-395), ops.gelu (src/ops.zig:310-340), ops.add,
// and Qwen2's ops.rmsNorm and ops.siluMul (src/ops.zig:409-439).
//
// layer_norm_kernel: one wave per row.  The row is read once into registers (n <= 2048 floats:
// 8 float4 per lane), then mean = sum / n, var = sum((x - mean)^2) / n (the reference's two
// passes, src/ops.zig:358-374), inv = 1 / sqrt(var + eps), out = fma((x - mean) * inv, w, b)
// (:376-380).  Wider rows loop over global memory in the same three passes.  Sums are reduced
// across the wave by butterfly, so their rounding order differs from the reference's 16-lane
// vector order (a few f32 ulps).
//
// gelu: ggml's tanh form, 0.5 x (1 + tanh(c (x + 0.044715 x^3))), tanh(u) = 1 - 2 / (1 + e^(2u)),
// c = sqrt(2 / pi) (src/ops.zig:312-327), each product and sum rounded in the reference's order
// (no contraction); e^x is the device's expf.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "elementwise.hpp"
#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

using zwg_ew::kNormRegs;
using zwg_ew::wave_sum;

// 4 waves per workgroup, one row per wave.
__global__ __launch_bounds__(256) void layer_norm_kernel(const float *x, const float *w, const float *b, float *out,
                                                         int32_t m, int32_t n, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float *xr = x + row * n;
    float *orow = out + row * n;
    const int n4 = n >> 2;
    const float fn = (float)n;
    if (n4 <= 64 * kNormRegs) {
        f32x4 v[kNormRegs];
#pragma unroll
        for (int i = 0; i < kNormRegs; ++i) {
            const int c = lane + 64 * i;
            v[i] = c < n4 ? reinterpret_cast<const f32x4 *>(xr)[c] : (f32x4){0.f, 0.f, 0.f, 0.f};
        }
        zwg_ew::layer_norm_regs<kNormRegs>(v, lane, n4, w, b, eps, orow);
        return;
    }
    float s = 0.f;
    for (int c = lane; c < n4; c += 64) {
        const f32x4 v = reinterpret_cast<const f32x4 *>(xr)[c];
        s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    const float mean = wave_sum(s) / fn;
    float q = 0.f;
    for (int c = lane; c < n4; c += 64) {
        const f32x4 v = reinterpret_cast<const f32x4 *>(xr)[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = v[e] - mean;
            q = __builtin_fmaf(d, d, q);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / fn + eps);
    for (int c = lane; c < n4; c += 64) {
        const f32x4 v = reinterpret_cast<const f32x4 *>(xr)[c];
        const f32x4 wv = reinterpret_cast<const f32x4 *>(w)[c];
        const f32x4 bv = reinterpret_cast<const f32x4 *>(b)[c];
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf((v[e] - mean) * inv, wv[e], bv[e]);
        reinterpret_cast<f32x4 *>(orow)[c] = o;
    }
}

// 4 waves per workgroup, one row per wave; ops.rmsNorm through zwg_ew::rms_norm_regs, wider rows
// in the same order over global memory.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *x, const float *w, float *out, int32_t m, int32_t n,
                                                       float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    const float *xr = x + row * n;
    float *orow = out + row * n;
    const int n4 = n >> 2;
    if (n4 <= 64 * kNormRegs) {
        f32x4 v[kNormRegs];
#pragma unroll
        for (int i = 0; i < kNormRegs; ++i) {
            const int c = lane + 64 * i;
            v[i] = c < n4 ? reinterpret_cast<const f32x4 *>(xr)[c] : (f32x4){0.f, 0.f, 0.f, 0.f};
        }
        zwg_ew::rms_norm_regs<kNormRegs>(v, lane, n4, w, eps, orow);
        return;
    }
    float q = 0.f;
    for (int c = lane; c < n4; c += 64) {
        const f32x4 v = reinterpret_cast<const f32x4 *>(xr)[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) q = __builtin_fmaf(v[e], v[e], q);
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float)n + eps);
    for (int c = lane; c < n4; c += 64) {
        const f32x4 v = reinterpret_cast<const f32x4 *>(xr)[c];
        const f32x4 wv = reinterpret_cast<const f32x4 *>(w)[c];
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
            const float r = v[e] * inv;
            o[e] = r * wv[e];
        }
        reinterpret_cast<f32x4 *>(orow)[c] = o;
    }
}

// ops.siluMul: gate = gate / (1 + e^-gate) * up
__global__ __launch_bounds__(256) void silu_mul_kernel(float *gate, const float *up, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        f32x4 g = reinterpret_cast<f32x4 *>(gate)[i];
        const f32x4 u = reinterpret_cast<const f32x4 *>(up)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] = zwg_ew::silu_mul(g[e], u[e]);
        reinterpret_cast<f32x4 *>(gate)[i] = g;
    }
}

__global__ __launch_bounds__(256) void gelu_kernel(float *x, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        f32x4 v = reinterpret_cast<f32x4 *>(x)[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = zwg_ew::gelu(v[e]);
        reinterpret_cast<f32x4 *>(x)[i] = v;
    }
}

__global__ __launch_bounds__(256) void add_kernel(float *x, const float *y, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        f32x4 v = reinterpret_cast<f32x4 *>(x)[i];
        const f32x4 u = reinterpret_cast<const f32x4 *>(y)[i];
        reinterpret_cast<f32x4 *>(x)[i] = v + u;
    }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

unsigned stride_grid(int64_t n4) { return (unsigned)std::min<int64_t>((n4 + 255) / 256, 256 * 8); }

} // namespace

namespace zwg_host {

int layer_norm(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, const float *b, float eps,
               float *out) {
    if (m == 0) return ZWG_OK;
    if (n == 0 || n % 4 || n > 0x7fffffffull || m > 0x7fffffffull) return fail(ctx, "n must be a positive multiple of 4");
    if (!x || !w || !b || !out) return fail(ctx, "null x, w, b or out");
    if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(out)) return fail(ctx, "buffers must be 16-byte aligned");
    layer_norm_kernel<<<(unsigned)((m + 3) / 4), 256, 0, ctx->stream>>>(x, w, b, out, (int32_t)m, (int32_t)n, eps);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ZWG_OK : fail_hip(ctx, "layer norm launch", e);
}

int rms_norm(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, float eps, float *out) {
    if (m == 0) return ZWG_OK;
    if (n == 0 || n % 4 || n > 0x7fffffffull || m > 0x7fffffffull) return fail(ctx, "n must be a positive multiple of 4");
    if (!x || !w || !out) return fail(ctx, "null x, w or out");
    if (!aligned16(x) || !aligned16(w) || !aligned16(out)) return fail(ctx, "buffers must be 16-byte aligned");
    rms_norm_kernel<<<(unsigned)((m + 3) / 4), 256, 0, ctx->stream>>>(x, w, out, (int32_t)m, (int32_t)n, eps);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? ZWG_OK : fail_hip(ctx, "rms norm launch", e);
}

} // namespace zwg_host

extern "C" {

int zwg_rms_norm_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, float eps, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    return rms_norm(ctx, x, m, n, w, eps, out);
}

int zwg_silu_mul_dev(zwg_ctx *ctx, float *gate, const float *up, uint64_t count) {
    if (!ctx) return fail(nullptr, "null context");
    if (count == 0) return ZWG_OK;
    if (!gate || !up || count % 4 || !aligned16(gate) || !aligned16(up))
        return fail(ctx, "gate and up must be 16-byte aligned and count a multiple of 4");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    silu_mul_kernel<<<stride_grid((int64_t)(count / 4)), 256, 0, ctx->stream>>>(gate, up, (int64_t)(count / 4));
    e = hipGetLastError();
    return e == hipSuccess ? ZWG_OK : fail_hip(ctx, "silu-mul launch", e);
}

int zwg_layer_norm_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, const float *b, float eps,
                       float *out) {
    if (!ctx) return fail(nullptr, "null context");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    return layer_norm(ctx, x, m, n, w, b, eps, out);
}

int zwg_gelu_dev(zwg_ctx *ctx, float *x, uint64_t count) {
    if (!ctx) return fail(nullptr, "null context");
    if (count == 0) return ZWG_OK;
    if (!x || count % 4 || !aligned16(x)) return fail(ctx, "x must be 16-byte aligned and count a multiple of 4");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    gelu_kernel<<<stride_grid((int64_t)(count / 4)), 256, 0, ctx->stream>>>(x, (int64_t)(count / 4));
    e = hipGetLastError();
    return e == hipSuccess ? ZWG_OK : fail_hip(ctx, "gelu launch", e);
}

int zwg_add_dev(zwg_ctx *ctx, float *x, const float *y, uint64_t count) {
    if (!ctx) return fail(nullptr, "null context");
    if (count == 0) return ZWG_OK;
    if (!x || !y || count % 4 || !aligned16(x) || !aligned16(y))
        return fail(ctx, "x and y must be 16-byte aligned and count a multiple of 4");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    add_kernel<<<stride_grid((int64_t)(count / 4)), 256, 0, ctx->stream>>>(x, y, (int64_t)(count / 4));
    e = hipGetLastError();
    return e == hipSuccess ? ZWG_OK : fail_hip(ctx, "add launch", e);
}

} // extern "C"
