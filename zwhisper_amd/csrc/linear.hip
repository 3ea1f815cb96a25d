// Linear layers around attention on gfx950 MFMA (include/zw_gpu.h, zwg_linear*).
//
// Replaces ops.linear (src/ops.zig:283-306) with f16 weights: out[i][o] = sum_p x[i][p] * w[o][p]
// (+ b[o]), x f32 [m][k], w f16 [n][k] (logically [n][k], as the reference keeps them), over the
// register-blocked broadcast-FMA kernels of src/gemm.zig:117-137 (ntBlock / micro4x4 / dot1).
// Callers: the encoder's Q/K/V/O projections and MLP (src/encoder.zig:164-174), BERT
// (src/bert.zig:223-232), the scene model (src/scene.zig:369-378).  The kernel, its precision
// and its tiling are described in linear_kernel.hpp.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "linear_kernel.hpp"
#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;
using zwg_lin::LinearArgs;

namespace {

int64_t tiles(uint64_t m, uint64_t n, int bm, int bn) { return (int64_t)((m + bm - 1) / bm) * (int64_t)((n + bn - 1) / bn); }

// Tile choice (swept on the device over the encoder, decoder and Qwen2 projection shapes): the
// 128 x 256 tile when it gives two workgroups per CU (256 CUs), else 64 x 256 when that fills
// the CUs once, else 64 x 64 for the small single-window shapes, which are latency bound.
hipError_t launch_linear(const LinearArgs &a, hipStream_t stream) {
    if (tiles(a.m, a.n, 128, 256) >= 512) return zwg_lin::launch_linear_tile<128, 256>(a, stream);
    if (tiles(a.m, a.n, 64, 256) >= 256) return zwg_lin::launch_linear_tile<64, 256>(a, stream);
    return zwg_lin::launch_linear_tile<64, 64>(a, stream);
}

std::string check_linear(uint64_t m, uint64_t k, uint32_t w_type, uint64_t n) {
    if (w_type != ZWG_W_F16) return "w_type must be ZWG_W_F16";
    if (k == 0 || k % 8) return "k must be a positive multiple of 8";
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return "m, n and k must be below 2^31";
    if ((n + 63) / 64 > 65535) return "n too large (above 65535 x 64)";
    if (k > (1ull << 20)) return "k above 2^20";  // keeps a workgroup's buffer range below 2^31 bytes
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
