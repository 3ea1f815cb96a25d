// Linear layers around attention on gfx950 MFMA (include/zw_gpu.h, zwg_linear*).
//
// Replaces ops.linear (src/ops.zig:283-306) with f16 weights: out[i][o] = sum_p x[i][p] * w[o][p]
// (+ b[o]), x f32 [m][k], w f16 [n][k] (logically [n][k], as the reference keeps them), over the
// register-blocked broadcast-FMA kernels of src/gemm.zig:117-137 (ntBlock / micro4x4 / dot1).
// Callers: the encoder's Q/K/V/O projections and MLP (src/encoder.zig:164-174), BERT
// (src/bert.zig:223-232), the scene model (src/scene.zig:369-378).
//
// Precision.  An f16 weight is exact in f16, and each f32 activation is split into two f16
// terms, x = hi + lo with hi = f16(x) and lo = f16(x - hi): they keep 22 of x's 24 significand
// bits, so the residual is below 2^-21 |x| (subnormal lo terms lose less than 2^-25 absolute).  Both products accumulate in f32 on
// v_mfma_f32_32x32x16_f16, so a dot product carries f32-level error, as the reference's f32
// FMA chain does, at the f16 MFMA rate.  |x| must stay within f16's range (65504); a larger
// input turns into inf in its output row rather than a wrong finite value.
//
// Tiles.  A workgroup of 4 waves computes a BM x BN block of out as 2 x 2 waves, each a
// (BM/2) x (BN/2) block of 32 x 32 MFMA tiles.  K goes through LDS 32 at a time, double-
// buffered: x converted to hi/lo f16 on its way in, w copied as is; rows padded by 8 halves
// so the 16-byte operand reads of a wave hit distinct banks.  MFMA operand layout (measured on
// the device): lane l, half s of A is A[l % 32][8 (l / 32) + s], of B is B[8 (l / 32) + s][l % 32];
// result register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BK = 32;      // K per LDS stage
constexpr int KPAD = BK + 8; // LDS row length in halves

struct LinearArgs {
    const float *x;         // [m][ldx]
    const _Float16 *w;      // [n][ldw]
    const float *bias;      // [n] or nullptr
    float *out;             // [m][ldo]
    int64_t ldx, ldw, ldo;
    int32_t m, n, k;
};

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void linear_f16_kernel(LinearArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2; // per wave
    constexpr int TM = WM / 32, TN = WN / 32; // 32 x 32 MFMA tiles per wave
    constexpr int XL = BM * BK / 4 / kThreads; // float4 loads of x per thread per stage
    constexpr int WL = BN * BK / 8 / kThreads; // 8-half loads of w per thread per stage
    static_assert(XL >= 1 && WL >= 1, "tile too small for the workgroup");

    __shared__ __align__(16) _Float16 xh[2][BM * KPAD];
    __shared__ __align__(16) _Float16 xl[2][BM * KPAD];
    __shared__ __align__(16) _Float16 ws[2][BN * KPAD];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;

    f32x4 xr[XL];
    half8 wr[WL];
    // stage loads: x element (row, 4 k) and w element (row, 8 k); rows or k past the end read 0
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int f = tid + kThreads * i;
            const int row = f / (BK / 4), kq = 4 * (f % (BK / 4));
            const int gm = m0 + row, gk = k0 + kq;
            xr[i] = gm < a.m && gk < a.k ? *reinterpret_cast<const f32x4 *>(a.x + (int64_t)gm * a.ldx + gk)
                                         : (f32x4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            const int f = tid + kThreads * i;
            const int row = f / (BK / 8), kq = 8 * (f % (BK / 8));
            const int gn = n0 + row, gk = k0 + kq;
            wr[i] = gn < a.n && gk < a.k ? *reinterpret_cast<const half8 *>(a.w + (int64_t)gn * a.ldw + gk)
                                         : (half8){0, 0, 0, 0, 0, 0, 0, 0};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int f = tid + kThreads * i;
            const int row = f / (BK / 4), kq = 4 * (f % (BK / 4));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v = xr[i][j];
                const _Float16 hi = (_Float16)v;
                xh[buf][row * KPAD + kq + j] = hi;
                xl[buf][row * KPAD + kq + j] = (_Float16)(v - (float)hi);
            }
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            const int f = tid + kThreads * i;
            const int row = f / (BK / 8), kq = 8 * (f % (BK / 8));
            *reinterpret_cast<half8 *>(&ws[buf][row * KPAD + kq]) = wr[i];
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (f32x16){0};

    const int n_k = (a.k + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    const int r32 = lane & 31, kh = 8 * (lane >> 5);
    for (int t = 0; t < n_k; ++t) {
        const int buf = t & 1;
        if (t + 1 < n_k) load((t + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            half8 ah[TM], al[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int row = wm * WM + i * 32 + r32;
                ah[i] = *reinterpret_cast<const half8 *>(&xh[buf][row * KPAD + kk + kh]);
                al[i] = *reinterpret_cast<const half8 *>(&xl[buf][row * KPAD + kk + kh]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int row = wn * WN + j * 32 + r32;
                b[j] = *reinterpret_cast<const half8 *>(&ws[buf][row * KPAD + kk + kh]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], acc[i][j], 0, 0, 0);
                }
        }
        if (t + 1 < n_k) store(buf ^ 1);
        __syncthreads();
    }

    // epilogue: register r of lane l is out[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] of its tile
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + r32;
        if (col >= a.n) continue;
        const float bj = a.bias ? a.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < a.m) a.out[(int64_t)row * a.ldo + col] = acc[i][j][r] + bj;
            }
    }
}

hipError_t launch_linear(const LinearArgs &a, hipStream_t stream) {
    // 128 x 128 blocks when they fill the machine (256 CUs), else 64 x 64
    const int64_t big = (int64_t)((a.m + 127) / 128) * ((a.n + 127) / 128);
    if (big >= 256) {
        dim3 grid((unsigned)((a.m + 127) / 128), (unsigned)((a.n + 127) / 128));
        linear_f16_kernel<128, 128><<<grid, kThreads, 0, stream>>>(a);
    } else {
        dim3 grid((unsigned)((a.m + 63) / 64), (unsigned)((a.n + 63) / 64));
        linear_f16_kernel<64, 64><<<grid, kThreads, 0, stream>>>(a);
    }
    return hipGetLastError();
}

std::string check_linear(uint64_t m, uint64_t k, uint32_t w_type, uint64_t n) {
    if (w_type != ZWG_W_F16) return "w_type must be ZWG_W_F16";
    if (k == 0 || k % 8) return "k must be a positive multiple of 8";
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return "m, n and k must be below 2^31";
    if ((m + 63) / 64 > 0x7fffffffull || (n + 63) / 64 > 65535) return "n too large";
    return "";
}

int run_linear(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
               const float *bias, uint64_t n, float *out) {
    const std::string msg = check_linear(m, k, w_type, n);
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0 || n == 0) return ZWG_OK;
    if (!x || !w || !out) return fail(ctx, "null x, w or out");
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(x) || !al16(w) || !al16(out)) return fail(ctx, "x, w and out must be 16-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    LinearArgs a{};
    a.x = x;
    a.w = static_cast<const _Float16 *>(w);
    a.bias = bias;
    a.out = out;
    a.ldx = (int64_t)k;
    a.ldw = (int64_t)k;
    a.ldo = (int64_t)n;
    a.m = (int32_t)m;
    a.n = (int32_t)n;
    a.k = (int32_t)k;
    e = launch_linear(a, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "linear kernel launch", e);
    return ZWG_OK;
}

} // namespace

extern "C" {

int zwg_linear_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
                   const float *bias, uint64_t n, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    return run_linear(ctx, x, m, k, w, w_type, bias, n, out);
}

int zwg_linear(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
               const float *bias, uint64_t n, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    const std::string msg = check_linear(m, k, w_type, n);
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0 || n == 0) return ZWG_OK;
    if (!x || !w || !out) return fail(ctx, "null x, w or out");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    // staging: x in slot 0, w in slot 1, bias then out in slots 2 and 3
    const uint64_t xb = m * k * 4, wb = n * k * 2, bb = bias ? n * 4 : 0, ob = m * n * 4;
    if (ensure_stage(ctx, 0, xb) || ensure_stage(ctx, 1, wb) || ensure_stage(ctx, 2, bb + 16) ||
        ensure_stage(ctx, 3, ob))
        return ZWG_ERROR;
    e = hipMemcpyAsync(ctx->stage[0], x, xb, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(ctx->stage[1], w, wb, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && bias) e = hipMemcpyAsync(ctx->stage[2], bias, bb, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipMemcpyAsync (linear upload)", e);
    int rc = run_linear(ctx, ctx->stage[0], m, k, ctx->stage[1], w_type, bias ? ctx->stage[2] : nullptr, n,
                        ctx->stage[3]);
    if (rc != ZWG_OK) return rc;
    e = hipMemcpyAsync(out, ctx->stage[3], ob, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "linear download", e);
    return ZWG_OK;
}

} // extern "C"
