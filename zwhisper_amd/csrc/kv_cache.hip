// Device-resident KV caches for the attention calls (include/zw_gpu.h, zwg_kv_*).
//
// The reference keeps its caches in host memory and fills them on the CPU:
//   - the Whisper decoder writes each new token's K and V projections straight into
//     row-major caches [n_ctx][n_state] (src/decoder.zig:39-42, :182-183) and projects a window's
//     cross K/V once (src/decoder.zig:151-159);
//   - Qwen2 rotates q and k with NeoX rotary positions (src/llm.zig:182-183, :221-238, tables
//     :128-137), scatters k into a transposed cache [n_head_kv][d][n_ctx] and copies v into
//     [n_ctx][n_head_kv*d] (src/llm.zig:185-190).
// Here the caches live in HBM, one per (layer, sequence), laid out [layer][sequence][...] so a
// batch of sequences is a zwg_batch at a fixed stride, and one kernel does an append: rotary
// positions on k (and q), the transposed scatter or the row copy of k, and the row copy of v.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;

namespace {

constexpr int kAppendThreads = 256;
// tokens per workgroup: 32 for one sequence's rows (the transposed scatter then writes 128
// contiguous bytes per dim row), 4 for one row per sequence (more workgroups; each token's
// writes land in its own sequence's cache anyway)
constexpr int kAppendTokensSeq = 32;
constexpr int kAppendTokensBatch = 4;

struct AppendArgs {
    const float *k_src; // [n][src_stride]: head h at columns h*d ..
    const float *v_src;
    int64_t src_stride;
    float *q; // [n][q_stride], n_head heads of d, rotated in place; nullptr: none
    int64_t q_stride;
    int32_t n_head;
    float *k_cache; // the layer's caches: sequence s at + s * per_seq
    float *v_cache;
    int64_t per_seq;
    const float *cos; // [n_ctx][d/2]; nullptr: no rotary positions
    const float *sin;
    const int32_t *pos_dev; // per-token positions (token i belongs to sequence seq0 + i); nullptr:
    int32_t seq0;           //   every token belongs to seq0, at positions pos0, pos0 + 1, ...
    int32_t pos0;
    int32_t n;
    int32_t n_ctx;
    int32_t n_head_kv;
    int32_t kt; // 1: k cache transposed [n_head_kv][d][n_ctx]
};

// Workgroup (x, y): tokens [x*TOK, x*TOK + TOK) and, for y < n_head_kv, KV head y -- its k rows
// staged in LDS (read with the head dims across threads), rotated there, then written with the
// cache's fast axis across threads (dims for the row-major cache, tokens for the transposed
// one), and its v rows copied straight through -- or, for y >= n_head_kv, query head
// y - n_head_kv rotated in place.
template <int D, int TOK>
__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(AppendArgs a) {
#pragma clang fp contract(off) // the rotation rounds each product and sum, as the reference does
    constexpr int HALF = D / 2;
    __shared__ float ks[TOK][D + 1];
    __shared__ int32_t tok_seq[TOK], tok_pos[TOK];

    const int tid = threadIdx.x;
    const int y = blockIdx.y;
    const int t0 = blockIdx.x * TOK;
    const int nt = min(TOK, a.n - t0);
    const int kvw = a.n_head_kv * D;

    if (tid < TOK) {
        int s = a.seq0, p = -1;
        if (tid < nt) {
            const int t = t0 + tid;
            s = a.pos_dev ? a.seq0 + t : a.seq0;
            p = a.pos_dev ? a.pos_dev[t] : a.pos0 + t;
        }
        // a position outside the cache is skipped: its row is neither rotated nor written
        tok_seq[tid] = s;
        tok_pos[tid] = p >= 0 && p < a.n_ctx ? p : -1;
    }

    if (y >= a.n_head_kv) {
        // rotate query head y - n_head_kv of the tile's tokens (src/llm.zig:182, :221-238), four
        // pairs (j .. j+3, j+d/2 .. j+d/2+3) per thread and iteration
        const int head = y - a.n_head_kv;
        __syncthreads();
        for (int idx = tid; idx < nt * (HALF / 4); idx += kAppendThreads) {
            const int i = idx / (HALF / 4), j = 4 * (idx - i * (HALF / 4));
            const int pos = tok_pos[i];
            if (pos < 0) continue;
            const float4 c = *reinterpret_cast<const float4 *>(a.cos + (int64_t)pos * HALF + j);
            const float4 s = *reinterpret_cast<const float4 *>(a.sin + (int64_t)pos * HALF + j);
            float *qr = a.q + (int64_t)(t0 + i) * a.q_stride + head * D;
            const float4 x0 = *reinterpret_cast<const float4 *>(qr + j);
            const float4 x1 = *reinterpret_cast<const float4 *>(qr + j + HALF);
            *reinterpret_cast<float4 *>(qr + j) =
                make_float4(x0.x * c.x - x1.x * s.x, x0.y * c.y - x1.y * s.y, x0.z * c.z - x1.z * s.z, x0.w * c.w - x1.w * s.w);
            *reinterpret_cast<float4 *>(qr + j + HALF) =
                make_float4(x0.x * s.x + x1.x * c.x, x0.y * s.y + x1.y * c.y, x0.z * s.z + x1.z * c.z, x0.w * s.w + x1.w * c.w);
        }
        return;
    }

    const int h = y;
    constexpr int D4 = D / 4;
    for (int idx = tid; idx < nt * D4; idx += kAppendThreads) {
        const int i = idx / D4, p = 4 * (idx - i * D4);
        const float4 x = *reinterpret_cast<const float4 *>(a.k_src + (int64_t)(t0 + i) * a.src_stride + h * D + p);
        ks[i][p] = x.x;
        ks[i][p + 1] = x.y;
        ks[i][p + 2] = x.z;
        ks[i][p + 3] = x.w;
    }
    __syncthreads();
    if (a.cos) {
        // NeoX pairs (j, j + d/2) at the token's position (src/llm.zig:221-238)
        for (int idx = tid; idx < nt * HALF; idx += kAppendThreads) {
            const int i = idx / HALF, j = idx - i * HALF;
            const int pos = tok_pos[i];
            if (pos < 0) continue;
            const float c = a.cos[(int64_t)pos * HALF + j], s = a.sin[(int64_t)pos * HALF + j];
            const float x0 = ks[i][j], x1 = ks[i][j + HALF];
            ks[i][j] = x0 * c - x1 * s;
            ks[i][j + HALF] = x0 * s + x1 * c;
        }
        __syncthreads();
    }
    if (a.kt) {
        // transposed: element (token i, dim p) at (h*D + p) * n_ctx + pos; tokens across threads
        for (int idx = tid; idx < nt * D; idx += kAppendThreads) {
            const int p = idx / nt, i = idx - p * nt;
            const int pos = tok_pos[i];
            if (pos < 0) continue;
            a.k_cache[(int64_t)tok_seq[i] * a.per_seq + (int64_t)(h * D + p) * a.n_ctx + pos] = ks[i][p];
        }
    } else {
        for (int idx = tid; idx < nt * D4; idx += kAppendThreads) {
            const int i = idx / D4, p = 4 * (idx - i * D4);
            const int pos = tok_pos[i];
            if (pos < 0) continue;
            *reinterpret_cast<float4 *>(a.k_cache + (int64_t)tok_seq[i] * a.per_seq + (int64_t)pos * kvw + h * D + p) =
                make_float4(ks[i][p], ks[i][p + 1], ks[i][p + 2], ks[i][p + 3]);
        }
    }
    for (int idx = tid; idx < nt * D4; idx += kAppendThreads) {
        const int i = idx / D4, p = 4 * (idx - i * D4);
        const int pos = tok_pos[i];
        if (pos < 0) continue;
        *reinterpret_cast<float4 *>(a.v_cache + (int64_t)tok_seq[i] * a.per_seq + (int64_t)pos * kvw + h * D + p) =
            *reinterpret_cast<const float4 *>(a.v_src + (int64_t)(t0 + i) * a.src_stride + h * D + p);
    }
}

hipError_t launch_append(const AppendArgs &a, int d, hipStream_t stream) {
    const int tok = a.pos_dev ? kAppendTokensBatch : kAppendTokensSeq;
    const int q_heads = a.q && a.cos ? a.n_head : 0;
    dim3 grid((unsigned)((a.n + tok - 1) / tok), (unsigned)(a.n_head_kv + q_heads));
#define ZWG_APPEND(DD)                                                                                           \
    if (a.pos_dev)                                                                                               \
        kv_append_kernel<DD, kAppendTokensBatch><<<grid, kAppendThreads, 0, stream>>>(a);                        \
    else                                                                                                         \
        kv_append_kernel<DD, kAppendTokensSeq><<<grid, kAppendThreads, 0, stream>>>(a);
    switch (d) {
    case 32: ZWG_APPEND(32) break;
    case 64: ZWG_APPEND(64) break;
    case 128: ZWG_APPEND(128) break;
    default: return hipErrorInvalidValue;
    }
#undef ZWG_APPEND
    return hipGetLastError();
}

std::string check_desc(const zwg_kv_desc &d) {
    if (d.reserved != 0) return "kv desc.reserved must be 0";
    if (d.layout != ZWG_KV_ROW && d.layout != ZWG_KV_KT) return "kv layout must be ZWG_KV_ROW or ZWG_KV_KT";
    if (d.d != 32 && d.d != 64 && d.d != 128) return "kv head dim d must be 32, 64 or 128";
    if (d.n_layer == 0 || d.n_seq == 0 || d.n_ctx == 0 || d.n_head_kv == 0)
        return "kv n_layer, n_seq, n_ctx and n_head_kv must be positive";
    if (d.n_ctx > 0x7fffffffull || d.n_seq > 0x7fffffffull || d.n_head_kv > 65535) return "kv sizes out of range";
    if (d.layout == ZWG_KV_KT && d.n_ctx % 4) return "a transposed key cache needs n_ctx a multiple of 4";
    if (!(d.rope_base >= 0.0) || std::isinf(d.rope_base)) return "rope_base must be finite and >= 0";
    return "";
}

// Rotary tables in f64, rounded to f32: angle = p / base^(2i/d) (src/llm.zig:128-137).
void rope_tables(const zwg_kv_desc &d, std::vector<float> &c, std::vector<float> &s) {
    const uint64_t half = d.d / 2;
    c.resize(d.n_ctx * half);
    s.resize(d.n_ctx * half);
    for (uint64_t i = 0; i < half; ++i) {
        const double inv = 1.0 / std::pow(d.rope_base, (double)(2 * i) / (double)d.d);
        for (uint64_t p = 0; p < d.n_ctx; ++p) {
            const double ang = (double)p * inv;
            c[p * half + i] = (float)std::cos(ang);
            s[p * half + i] = (float)std::sin(ang);
        }
    }
}

// Shared body of the append calls: validate, stage host rows if asked, launch.
int append(zwg_kv *kv, uint64_t layer, uint64_t seq0, uint64_t pos0, uint64_t n, const int32_t *pos_dev,
           const float *k_rows, const float *v_rows, float *q, uint64_t n_head, uint64_t q_stride, uint32_t flags) {
    zwg_ctx *ctx = kv->ctx;
    const zwg_kv_desc &d = kv->desc;
    if (flags & ~ZWG_ROWS_ON_HOST) return fail(ctx, "unknown kv append flags");
    if (layer >= d.n_layer) return fail(ctx, "kv layer out of range");
    if (n == 0) return ZWG_OK;
    if (!k_rows || !v_rows) return fail(ctx, "null k or v rows");
    if (n > 0x7fffffffull) return fail(ctx, "too many rows");
    if (pos_dev) {
        if (seq0 + n > d.n_seq) return fail(ctx, "kv sequences out of range");
        if (flags & ZWG_ROWS_ON_HOST) return fail(ctx, "per-sequence positions are a device array: no host rows");
    } else {
        if (seq0 >= d.n_seq) return fail(ctx, "kv sequence out of range");
        if (pos0 + n > d.n_ctx) return fail(ctx, "append past the end of the cache (pos + n > n_ctx)");
    }
    if (q) {
        if (d.rope_base <= 0.0) return fail(ctx, "q is rotated only when the cache has rope_base > 0");
        if (n_head == 0 || n_head % d.n_head_kv) return fail(ctx, "n_head must be a positive multiple of n_head_kv");
        if (n_head + d.n_head_kv > 65535) return fail(ctx, "n_head out of range");
        if (q_stride < n_head * d.d) return fail(ctx, "q_stride is smaller than n_head * d");
    }
    if (!(flags & ZWG_ROWS_ON_HOST)) {
        const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
        if (!al16(k_rows) || !al16(v_rows) || (q && !al16(q))) return fail(ctx, "k, v and q rows must be 16-byte aligned");
    }
    if (q && q_stride % 4) return fail(ctx, "q_stride must be a multiple of 4 floats");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    const uint64_t F = sizeof(float);
    const float *ks = k_rows, *vs = v_rows;
    float *qd = q;
    if (flags & ZWG_ROWS_ON_HOST) {
        const uint64_t rows = n * kv->kvw * F, qrows = q ? ((n - 1) * q_stride + n_head * d.d) * F : 0;
        if (ensure_stage(ctx, 1, rows) || ensure_stage(ctx, 2, rows) || (q && ensure_stage(ctx, 0, qrows)))
            return ZWG_ERROR;
        e = hipMemcpyAsync(ctx->stage[1], k_rows, rows, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(ctx->stage[2], v_rows, rows, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess && q) e = hipMemcpyAsync(ctx->stage[0], q, qrows, hipMemcpyHostToDevice, ctx->stream);
        if (e != hipSuccess) return fail_hip(ctx, "hipMemcpyAsync (kv rows upload)", e);
        ks = ctx->stage[1];
        vs = ctx->stage[2];
        qd = q ? ctx->stage[0] : nullptr;
    }
    AppendArgs a{};
    a.k_src = ks;
    a.v_src = vs;
    a.src_stride = (int64_t)kv->kvw;
    a.q = qd;
    a.q_stride = (int64_t)q_stride;
    a.n_head = (int32_t)n_head;
    a.k_cache = kv->k + layer * d.n_seq * kv->per_seq;
    a.v_cache = kv->v + layer * d.n_seq * kv->per_seq;
    a.per_seq = (int64_t)kv->per_seq;
    a.cos = kv->cos;
    a.sin = kv->sin;
    a.pos_dev = pos_dev;
    a.seq0 = (int32_t)seq0;
    a.pos0 = (int32_t)pos0;
    a.n = (int32_t)n;
    a.n_ctx = (int32_t)d.n_ctx;
    a.n_head_kv = (int32_t)d.n_head_kv;
    a.kt = d.layout == ZWG_KV_KT;
    e = launch_append(a, (int)d.d, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "kv append kernel launch", e);
    if (flags & ZWG_ROWS_ON_HOST) {
        if (q) {
            // hand the rotated q back, as src/llm.zig:182 rotates the caller's q in place
            const uint64_t qrows = ((n - 1) * q_stride + n_head * d.d) * F;
            e = hipMemcpyAsync(q, qd, qrows, hipMemcpyDeviceToHost, ctx->stream);
            if (e != hipSuccess) return fail_hip(ctx, "hipMemcpyAsync (q download)", e);
        }
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return fail_hip(ctx, "hipStreamSynchronize", e);
    }
    return ZWG_OK;
}

} // namespace

namespace {

const char *const kKvClosed = "the kv cache's context is closed";

// Free a cache's device memory (after the work queued on its context's stream).
void free_caches(zwg_kv *kv) {
    (void)hipSetDevice(kv->ctx->device);
    (void)hipStreamSynchronize(kv->ctx->stream);
    for (float **p : {&kv->k, &kv->v, &kv->cos, &kv->sin}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
}

// zwg_close of the cache's context: the caches go with it
void detach_kv(void *obj) {
    auto *kv = static_cast<zwg_kv *>(obj);
    free_caches(kv);
    kv->ctx = nullptr;
}

} // namespace

extern "C" {

int zwg_kv_create(zwg_ctx *ctx, const zwg_kv_desc *desc, zwg_kv **out) {
    if (!out) return fail(ctx, "null output pointer");
    *out = nullptr;
    if (!ctx || !desc) return fail(ctx, "null context or kv desc");
    const std::string msg = check_desc(*desc);
    if (!msg.empty()) return fail(ctx, msg);
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    zwg_kv *kv = new zwg_kv();
    kv->ctx = ctx;
    kv->desc = *desc;
    kv->kvw = desc->n_head_kv * desc->d;
    kv->per_seq = desc->n_ctx * kv->kvw;
    const uint64_t bytes = desc->n_layer * desc->n_seq * kv->per_seq * sizeof(float);
    void *pk = nullptr, *pv = nullptr;
    e = hipMalloc(&pk, bytes);
    if (e == hipSuccess) e = hipMalloc(&pv, bytes);
    // zero, as the reference's transposed cache is (src/llm.zig:125): columns at and past n_kv
    // of a K^T row must hold finite values
    if (e == hipSuccess) e = hipMemsetAsync(pk, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(pv, 0, bytes, ctx->stream);
    kv->k = static_cast<float *>(pk);
    kv->v = static_cast<float *>(pv);
    if (e == hipSuccess && desc->rope_base > 0.0) {
        std::vector<float> c, s;
        rope_tables(*desc, c, s);
        const uint64_t tb = c.size() * sizeof(float);
        void *pc = nullptr, *ps = nullptr;
        e = hipMalloc(&pc, tb);
        if (e == hipSuccess) e = hipMalloc(&ps, tb);
        kv->cos = static_cast<float *>(pc);
        kv->sin = static_cast<float *>(ps);
        if (e == hipSuccess) e = hipMemcpyAsync(pc, c.data(), tb, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(ps, s.data(), tb, hipMemcpyHostToDevice, ctx->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        free_caches(kv);
        delete kv;
        return fail_hip(ctx, "kv cache allocation", e);
    }
    add_child(ctx, kv, detach_kv);
    *out = kv;
    return ZWG_OK;
}

void zwg_kv_destroy(zwg_kv *kv) {
    if (!kv) return;
    if (kv->ctx) {
        remove_child(kv->ctx, kv);
        free_caches(kv);
    }
    delete kv;
}

int zwg_kv_get_info(const zwg_kv *kv, zwg_kv_info *out) {
    if (!kv || !out) return fail(kv ? kv->ctx : nullptr, "null kv or output");
    if (!kv->ctx) return fail(nullptr, kKvClosed);
    out->k = kv->k;
    out->v = kv->v;
    out->layer_stride = kv->desc.n_seq * kv->per_seq;
    out->seq_stride = kv->per_seq;
    out->kv_stride = kv->kvw;
    out->kt_stride = kv->desc.layout == ZWG_KV_KT ? kv->desc.n_ctx : 0;
    return ZWG_OK;
}

int zwg_kv_append(zwg_kv *kv, uint64_t layer, uint64_t seq, uint64_t pos, uint64_t n, const float *k_rows,
                  const float *v_rows, float *q, uint64_t n_head, uint64_t q_stride, uint32_t flags) {
    if (!kv) return fail(nullptr, "null kv");
    if (!kv->ctx) return fail(nullptr, kKvClosed);
    return append(kv, layer, seq, pos, n, nullptr, k_rows, v_rows, q, n_head, q_stride, flags);
}

int zwg_kv_append_batch(zwg_kv *kv, uint64_t layer, uint64_t seq0, uint64_t n_seq, const int32_t *pos_dev,
                        const float *k_rows, const float *v_rows, float *q, uint64_t n_head, uint64_t q_stride) {
    if (!kv) return fail(nullptr, "null kv");
    if (!kv->ctx) return fail(nullptr, kKvClosed);
    if (!pos_dev) return fail(kv->ctx, "null position array");
    return append(kv, layer, seq0, 0, n_seq, pos_dev, k_rows, v_rows, q, n_head, q_stride, 0);
}

int zwg_kv_read(zwg_kv *kv, uint64_t layer, uint64_t seq, float *k_host, float *v_host) {
    if (!kv) return fail(nullptr, "null kv");
    if (!kv->ctx) return fail(nullptr, kKvClosed);
    zwg_ctx *ctx = kv->ctx;
    if (layer >= kv->desc.n_layer || seq >= kv->desc.n_seq) return fail(ctx, "kv layer or sequence out of range");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    const uint64_t off = (layer * kv->desc.n_seq + seq) * kv->per_seq, bytes = kv->per_seq * sizeof(float);
    if (k_host) e = hipMemcpyAsync(k_host, kv->k + off, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess && v_host) e = hipMemcpyAsync(v_host, kv->v + off, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "kv read", e);
    return ZWG_OK;
}

} // extern "C"
