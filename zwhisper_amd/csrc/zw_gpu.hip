// C ABI of the attention library (include/zw_gpu.h): contexts, shape checks, planning and
// dispatch to the dense MFMA kernel (attn_flash.hip) or the split-K decode kernel
// (attn_decode.hip).
#include "zw_gpu.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "attn_kernels.hpp"
#include "attn_plan.hpp"
#include "zw_ctx.hpp"

namespace zwg_host {

thread_local std::string t_err;

int fail(zwg_ctx *ctx, const std::string &msg) {
    t_err = msg;
    if (ctx) ctx->err = msg;
    return ZWG_ERROR;
}

int fail_hip(zwg_ctx *ctx, const char *what, hipError_t e) {
    return fail(ctx, std::string(what) + ": " + hipGetErrorString(e));
}

int ensure_stage(zwg_ctx *ctx, int i, uint64_t bytes) {
    bytes = std::max<uint64_t>(bytes, 256);
    if (ctx->stage_bytes[i] >= bytes) return ZWG_OK;
    if (ctx->fixed_staging) {
        char buf[200];
        snprintf(buf, sizeof buf, "this call needs %llu bytes of staging, more than the context's staging_bytes (%llu)",
                 (unsigned long long)bytes, (unsigned long long)ctx->stage_bytes[i]);
        return fail(ctx, buf);
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipStreamSynchronize", e);
    if (ctx->stage[i]) {
        (void)hipFree(ctx->stage[i]);
        ctx->stage[i] = nullptr;
        ctx->stage_bytes[i] = 0;
    }
    void *p = nullptr;
    e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail_hip(ctx, "hipMalloc (staging)", e);
    ctx->stage[i] = static_cast<float *>(p);
    ctx->stage_bytes[i] = bytes;
    return ZWG_OK;
}

int download_rows(zwg_ctx *ctx, float *dst, const float *src, uint64_t n_rows, uint64_t cols, uint64_t stride) {
    const uint64_t F = sizeof(float);
    if (n_rows == 0) return ZWG_OK;
    hipError_t e;
    if (stride == cols || n_rows == 1) {
        e = hipMemcpyAsync(dst, src, ((n_rows - 1) * stride + cols) * F, hipMemcpyDeviceToHost, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return fail_hip(ctx, "download", e);
        return ZWG_OK;
    }
    const uint64_t span = ((n_rows - 1) * stride + cols) * F;
    if (ctx->host_stage_bytes < span && ctx->fixed_staging) {
        char buf[200];
        snprintf(buf, sizeof buf,
                 "this call's result needs %llu bytes of pinned host staging, more than the context's staging_bytes "
                 "(%llu)", (unsigned long long)span, (unsigned long long)ctx->host_stage_bytes);
        return fail(ctx, buf);
    }
    if (ctx->host_stage_bytes < span) {
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return fail_hip(ctx, "hipStreamSynchronize", e);
        if (ctx->host_stage) (void)hipHostFree(ctx->host_stage);
        ctx->host_stage = nullptr;
        ctx->host_stage_bytes = 0;
        void *p = nullptr;
        e = hipHostMalloc(&p, span, hipHostMallocDefault);
        if (e != hipSuccess) return fail_hip(ctx, "hipHostMalloc (result staging)", e);
        ctx->host_stage = static_cast<float *>(p);
        ctx->host_stage_bytes = span;
    }
    e = hipMemcpyAsync(ctx->host_stage, src, span, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "download", e);
    for (uint64_t r = 0; r < n_rows; ++r) std::memcpy(dst + r * stride, ctx->host_stage + r * stride, cols * F);
    return ZWG_OK;
}

void add_child(zwg_ctx *ctx, void *obj, void (*detach)(void *)) { ctx->children.push_back({obj, detach}); }

void remove_child(zwg_ctx *ctx, void *obj) {
    auto &c = ctx->children;
    for (size_t i = 0; i < c.size(); ++i)
        if (c[i].obj == obj) {
            c.erase(c.begin() + (ptrdiff_t)i);
            return;
        }
}

} // namespace zwg_host

using namespace zwg_host;

namespace {

using namespace zwg_planner;

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Where and how a call runs: the context's device, stream, workspace and dense mode, or, for the
// allocation-free entry point, the caller's stream and the library's static scratch.
struct Exec {
    int device;       // hipSetDevice first; -1: the calling thread's current device
    hipStream_t stream;
    float *ws;        // split partials
    uint64_t ws_bytes;
    uint32_t dense_math;
    uint64_t plan_cap; // workspace bytes the planner may use (>= ws_bytes: a bigger plan is refused)
    const char *ws_name;
    uint32_t *out_max = nullptr; // device words the kernels raise to the largest |out| they write, or null
    // K and V as tile images (the encoder layer's projections write them), read by the dense x3
    // kernel in place of k and v
    const _Float16 *k_img = nullptr, *v_img = nullptr;
    uint64_t img_tiles = 0;
    // q as q_parts k-split partials of its projection (AttnArgs::q_parts), decode kernels only
    int32_t q_parts = 0;
    int64_t q_part_stride = 0;
    const float *q_bias = nullptr;
};

Exec ctx_exec(const zwg_ctx *ctx) {
    return Exec{ctx->device, ctx->stream, ctx->workspace, ctx->workspace_bytes, ctx->dense_math,
                ctx->workspace_bytes, "the context's workspace"};
}

// The plan and the launches of a checked call whose head dim has kernels (32, 64, 128); scale is
// f32(1/sqrt(d)) of the caller's head dim.  ctx (may be null) receives the error.
int run_kernels(zwg_ctx *ctx, const Exec &x, const float *q, const float *k, const float *v, const zwg_attn_shape &s,
                const zwg_batch &b, float *out, Plan *plan_out, float scale) {
    const Plan p = make_plan(s, b, x.plan_cap, x.dense_math);
    if (plan_out) *plan_out = p;
    if (p.ws_bytes > x.ws_bytes) {
        char buf[200];
        snprintf(buf, sizeof buf, "this call's split partials need %llu bytes, more than the %llu bytes of %s",
                 (unsigned long long)p.ws_bytes, (unsigned long long)x.ws_bytes, x.ws_name);
        return fail(ctx, buf);
    }
    // the row-major decode kernel and both dense kernels (x3 and fp32) address one item's K/V rows
    // (and the dense kernels one KV head's K^T rows) through buffer descriptors with 32-bit byte
    // offsets; the dense kernels' tile loads reach up to 32 rows past the last key
    const bool dense = p.kernel == 1;
    if (x.k_img) {
        if (!dense || x.dense_math != ZWG_DENSE_X3 || s.kt_stride || (s.d != 64 && s.d != 128) ||
            x.img_tiles != (s.n_kv + 31) / 32 || b.n_kv_dev)
            return fail(ctx, "tile images are read by the dense x3 kernel only (row-major K, d 64 or 128, "
                             "all items at n_kv keys)");
        if (b.n_batch * s.n_head_kv * x.img_tiles * 64 * s.d * 2 > 0xffffffffffffull ||
            x.img_tiles * 64 * s.d * 2 > 0x7fffffffull)
            return fail(ctx, "tile images too large");
    } else if (x.q_parts > 1 && p.kernel != 2) {
        return fail(ctx, "queries as projection partials are read by the decode kernels only");
    } else if ((p.kernel == 2 && !s.kt_stride) || dense) {
        if (s.n_kv > 0 && ((s.n_kv - 1 + (dense ? 32 : 0)) * s.kv_stride + s.d) * sizeof(float) > 0x7fffffffull)
            return fail(ctx, "K/V rows of one batch item must span less than 2 GiB");
        if (dense && s.kt_stride && (s.d * s.kt_stride + 32) * sizeof(float) > 0x7fffffffull)
            return fail(ctx, "the transposed K rows of one KV head must span less than 2 GiB");
    }

    zwg::AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.q_stride = (int64_t)s.q_stride;
    a.kv_stride = (int64_t)s.kv_stride;
    a.out_stride = (int64_t)s.out_stride;
    a.kt_stride = (int64_t)s.kt_stride;
    a.q_bstride = (int64_t)b.q_bstride;
    a.k_bstride = (int64_t)b.k_bstride;
    a.v_bstride = (int64_t)b.v_bstride;
    a.out_bstride = (int64_t)b.out_bstride;
    a.n_kv_item = b.n_kv_dev;
    a.n_q = (int32_t)s.n_q;
    a.n_kv = (int32_t)s.n_kv;
    a.n_head = (int32_t)s.n_head;
    a.n_head_kv = (int32_t)s.n_head_kv;
    a.group = (int32_t)(s.n_head / s.n_head_kv);
    a.n_batch = (int32_t)b.n_batch;
    a.causal = s.causal ? 1 : 0;
    a.scale_log2 = scale * 1.4426950408889634f; // log2 units
    a.split_tile = p.split_tile;
    a.chunk_len = p.chunk_len;
    a.max_chunks = p.max_chunks;
    a.heavy_first = p.heavy_first;
    a.xcd_group = p.xcd_group;
    a.rows_per_unit = p.rows_per_unit;
    a.live_blocks = (int64_t)p.grid_blocks;
    const uint64_t n_rows = b.n_batch * s.n_head * s.n_q;
    a.part_ml = x.ws;
    a.part_o = x.ws + (p.max_chunks > 1 ? part_o_offset(n_rows, (uint64_t)p.max_chunks) : 0);
    a.out_max = x.out_max;
    a.k_img = x.k_img;
    a.v_img = x.v_img;
    a.img_tiles = (int32_t)x.img_tiles;
    a.q_parts = x.q_parts;
    a.q_part_stride = x.q_part_stride;
    a.q_bias = x.q_bias;

    hipError_t e = hipSuccess;
    if (x.device >= 0) e = hipSetDevice(x.device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    int blocks = 0;
    if (p.kernel == 1)
        e = x.dense_math == ZWG_DENSE_FP32 ? zwg::launch_flash(a, (int)s.d, x.stream, &blocks)
                                            : zwg::launch_flash_x3(a, (int)s.d, x.stream, &blocks);
    else if (p.kernel == 3)
        e = zwg::launch_generic(a, (int)s.d, x.stream);
    else
        e = zwg::launch_decode(a, (int)s.d, (int)(s.n_q * a.group), x.stream, &blocks);
    if (e != hipSuccess) return fail_hip(ctx, "attention kernel launch", e);
    if (p.max_chunks > 1) {
        e = zwg::launch_combine(a, (int)s.d, x.stream);
        if (e != hipSuccess) return fail_hip(ctx, "combine kernel launch", e);
    }
    return ZWG_OK;
}

// Shape and pointer checks, then the call on the kernels: directly for the built head dims, else
// over zero-padded copies in the context's staging (attn_pad.hip).  ctx (may be null) receives
// the error.
int run(zwg_ctx *ctx, const Exec &x, const float *q, const float *k, const float *v, const zwg_attn_shape &s,
        const zwg_batch &b, float *out, Plan *plan_out = nullptr) {
    std::string msg = check_shape(s);
    if (msg.empty()) msg = check_batch(s, b);
    if (!msg.empty()) return fail(ctx, msg);
    if (s.n_q == 0) return ZWG_OK;
    if (!q || !out || (s.n_kv && (!k || !v))) return fail(ctx, "null tensor pointer");
    if (!aligned16(q) || !aligned16(out) || (s.n_kv && (!aligned16(k) || !aligned16(v))))
        return fail(ctx, "q, k, v and out must be 16-byte aligned");
    // f32(1/sqrt(d)) as the reference computes it (src/ops.zig:531), of the caller's d
    const float scale = 1.0f / std::sqrt((float)s.d);
    const uint64_t D = kernel_d(s.d);
    if (D == s.d) return run_kernels(ctx, x, q, k, v, s, b, out, plan_out, scale); // built dims, and above 128
    if (!ctx)
        return fail(nullptr, "head dims other than 32, 64 and 128 run over zero-padded copies, which need a context "
                             "(zwg_attention_batch_dev)");

    // the same call at head dim D: q, v, out as [item][row][head][D], K row-major likewise or
    // transposed as [item][KV head][D][kt_stride]
    const uint64_t H = s.n_head, Hk = s.n_head_kv, B = b.n_batch;
    zwg_attn_shape s2 = s;
    s2.d = D;
    s2.q_stride = H * D;
    s2.out_stride = H * D;
    s2.kv_stride = Hk * D;
    zwg_batch b2 = b;
    b2.q_bstride = s.n_q * H * D;
    b2.out_bstride = s.n_q * H * D;
    b2.k_bstride = s.kt_stride ? Hk * D * s.kt_stride : s.n_kv * Hk * D;
    b2.v_bstride = s.n_kv * Hk * D;
    const uint64_t F = sizeof(float);
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    if (ensure_stage(ctx, 4, B * b2.q_bstride * F) || ensure_stage(ctx, 5, (B * b2.k_bstride + 4) * F) ||
        ensure_stage(ctx, 6, (B * b2.v_bstride + 4) * F) || ensure_stage(ctx, 7, B * b2.out_bstride * F))
        return ZWG_ERROR;
    float *qp = ctx->stage[4], *kp = ctx->stage[5], *vp = ctx->stage[6], *op = ctx->stage[7];
    const int d = (int)s.d, Di = (int)D;
    e = zwg::launch_pad_rows(q, qp, (int)B, (int)s.n_q, (int)H, d, Di, (int64_t)s.q_stride, (int64_t)b.q_bstride,
                             nullptr, x.stream);
    if (e == hipSuccess && s.n_kv) {
        if (s.kt_stride)
            e = zwg::launch_pad_kt(k, kp, (int)B, (int)Hk, d, Di, (int)s.kt_stride, (int)s.n_kv, (int64_t)b.k_bstride,
                                   b.n_kv_dev, x.stream);
        else
            e = zwg::launch_pad_rows(k, kp, (int)B, (int)s.n_kv, (int)Hk, d, Di, (int64_t)s.kv_stride,
                                     (int64_t)b.k_bstride, b.n_kv_dev, x.stream);
        if (e == hipSuccess)
            e = zwg::launch_pad_rows(v, vp, (int)B, (int)s.n_kv, (int)Hk, d, Di, (int64_t)s.kv_stride,
                                     (int64_t)b.v_bstride, b.n_kv_dev, x.stream);
    }
    if (e != hipSuccess) return fail_hip(ctx, "head-dim padding launch", e);
    const int rc = run_kernels(ctx, x, qp, kp, vp, s2, b2, op, plan_out, scale);
    if (rc != ZWG_OK) return rc;
    e = zwg::launch_unpad_rows(op, out, (int)B, (int)s.n_q, (int)H, d, Di, (int64_t)s.out_stride,
                               (int64_t)b.out_bstride, x.stream);
    if (e != hipSuccess) return fail_hip(ctx, "head-dim unpadding launch", e);
    return ZWG_OK;
}

} // namespace

int zwg_host::attention_images_dev(zwg_ctx *ctx, const float *q, const void *k_img, const void *v_img,
                                   uint64_t img_tiles, const zwg_attn_shape &s, const zwg_batch &b, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    if (!k_img || !v_img) return fail(ctx, "null tile image");
    Exec x = ctx_exec(ctx);
    x.k_img = static_cast<const _Float16 *>(k_img);
    x.v_img = static_cast<const _Float16 *>(v_img);
    x.img_tiles = img_tiles;
    return run(ctx, x, q, static_cast<const float *>(k_img), static_cast<const float *>(v_img), s, b, out);
}

int zwg_host::attention_qparts_dev(zwg_ctx *ctx, const float *q_parts, int n_parts, uint64_t part_stride,
                                   const float *q_bias, const float *k, const float *v, const zwg_attn_shape &s,
                                   const zwg_batch &b, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    if (n_parts < 2 || n_parts > zwg::kMaxQParts || part_stride > 0x7fffffffffffull)
        return fail(ctx, "q partials: two to eight, bounded stride");
    if (kernel_d(s.d) != s.d) return fail(ctx, "q partials need a head dim with kernels of its own (32, 64, 128)");
    Exec x = ctx_exec(ctx);
    x.q_parts = n_parts;
    x.q_part_stride = (int64_t)part_stride;
    x.q_bias = q_bias;
    return run(ctx, x, q_parts, k, v, s, b, out);
}

extern "C" {

int zwg_version(void) { return ZWG_VERSION; }

const char *zwg_last_error(const zwg_ctx *ctx) { return ctx ? ctx->err.c_str() : t_err.c_str(); }

int zwg_check_shape(const zwg_attn_shape *shape, char *msg, size_t msg_len) {
    if (!shape) {
        if (msg && msg_len) snprintf(msg, msg_len, "null shape");
        return ZWG_ERROR;
    }
    const std::string m = check_shape(*shape);
    if (msg && msg_len) snprintf(msg, msg_len, "%s", m.c_str());
    return m.empty() ? ZWG_OK : ZWG_ERROR;
}

int zwg_plan(const zwg_attn_shape *shape, const zwg_batch *batch, uint64_t workspace_bytes, zwg_plan_info *out) {
    if (!shape || !out) return fail(nullptr, "null argument");
    zwg_batch one{1, 0, 0, 0, 0, nullptr};
    const zwg_batch &b = batch ? *batch : one;
    std::string msg = check_shape(*shape);
    if (msg.empty()) msg = check_batch(*shape, b);
    if (!msg.empty()) return fail(nullptr, msg);
    const Plan p = make_plan(*shape, b, workspace_bytes ? workspace_bytes : kDefaultWorkspace, ZWG_DENSE_X3);
    out->kernel = (uint32_t)p.kernel;
    out->rows_per_unit = (uint32_t)p.rows_per_unit;
    out->chunk_len = (uint64_t)p.chunk_len;
    out->max_chunks = (uint64_t)p.max_chunks;
    out->grid_blocks = p.grid_blocks;
    out->workspace_bytes = p.ws_bytes;
    return ZWG_OK;
}

int zwg_open(int device, const zwg_limits *limits, zwg_ctx **out) {
    if (!out) return fail(nullptr, "null output pointer");
    *out = nullptr;
    int n_dev = 0;
    hipError_t e = hipGetDeviceCount(&n_dev);
    if (e != hipSuccess || n_dev == 0) return fail(nullptr, "no HIP device available");
    if (device < 0 || device >= n_dev) return fail(nullptr, "device index out of range");
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail_hip(nullptr, "hipSetDevice", e);
    zwg_ctx *ctx = new zwg_ctx();
    ctx->device = device;
    e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail_hip(nullptr, "hipStreamCreate", e);
    }
    ctx->stream = ctx->own_stream;
    ctx->workspace_bytes = (limits && limits->workspace_bytes) ? limits->workspace_bytes : kDefaultWorkspace;
    if (limits && limits->dense_math > ZWG_DENSE_FP32) {
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return fail(nullptr, "unknown dense_math");
    }
    ctx->dense_math = limits ? limits->dense_math : ZWG_DENSE_X3;
    e = hipEventCreateWithFlags(&ctx->switch_event, hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return fail_hip(nullptr, "hipEventCreate", e);
    }
    void *ws = nullptr;
    e = hipMalloc(&ws, ctx->workspace_bytes);
    if (e != hipSuccess) {
        (void)hipEventDestroy(ctx->switch_event);
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return fail_hip(nullptr, "hipMalloc (workspace)", e);
    }
    ctx->workspace = static_cast<float *>(ws);
    void *flag = nullptr;
    e = hipMalloc(&flag, zwg::kOutMaxBytes);
    if (e != hipSuccess) {
        (void)hipFree(ws);
        (void)hipEventDestroy(ctx->switch_event);
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return fail_hip(nullptr, "hipMalloc (flag)", e);
    }
    ctx->out_max_word = static_cast<uint32_t *>(flag);
    if (limits && limits->staging_bytes) {
        // every staging buffer at its fixed size now: no later call allocates
        const uint64_t sb = std::max<uint64_t>(limits->staging_bytes, 256);
        for (int i = 0; i < 8 && e == hipSuccess; ++i) {
            void *p = nullptr;
            e = hipMalloc(&p, sb);
            if (e == hipSuccess) {
                ctx->stage[i] = static_cast<float *>(p);
                ctx->stage_bytes[i] = sb;
            }
        }
        if (e == hipSuccess) {
            void *p = nullptr;
            e = hipHostMalloc(&p, sb, hipHostMallocDefault);
            if (e == hipSuccess) {
                ctx->host_stage = static_cast<float *>(p);
                ctx->host_stage_bytes = sb;
            }
        }
        ctx->fixed_staging = true;
        if (e != hipSuccess) {
            zwg_close(ctx);
            return fail_hip(nullptr, "allocating the staging buffers (zwg_limits.staging_bytes)", e);
        }
    }
    *out = ctx;
    return ZWG_OK;
}

int zwg_set_dense_math(zwg_ctx *ctx, uint32_t mode) {
    if (!ctx) return fail(nullptr, "null context");
    if (mode > ZWG_DENSE_FP32) return fail(ctx, "unknown dense math mode");
    ctx->dense_math = mode;
    return ZWG_OK;
}

void zwg_close(zwg_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    // objects made from this context and not destroyed yet lose their device memory now
    const std::vector<ZwgChild> children = ctx->children;
    for (const ZwgChild &c : children) c.detach(c.obj);
    ctx->children.clear();
    for (auto &s : ctx->stage)
        if (s) (void)hipFree(s);
    if (ctx->host_stage) (void)hipHostFree(ctx->host_stage);
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    if (ctx->out_max_word) (void)hipFree(ctx->out_max_word);
    if (ctx->switch_event) (void)hipEventDestroy(ctx->switch_event);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

int zwg_set_stream(zwg_ctx *ctx, void *hip_stream) {
    if (!ctx) return fail(nullptr, "null context");
    hipStream_t next = static_cast<hipStream_t>(hip_stream);
    if (next == ctx->stream) return ZWG_OK;
    // every call of the context writes the same workspace (split partials, staging), so work
    // queued on the new stream waits for what is already queued on the old one
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipEventRecord(ctx->switch_event, ctx->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(next, ctx->switch_event, 0);
    if (e != hipSuccess) return fail_hip(ctx, "stream switch ordering", e);
    ctx->stream = next;
    return ZWG_OK;
}

void *zwg_get_stream(const zwg_ctx *ctx) { return ctx ? static_cast<void *>(ctx->stream) : nullptr; }

int zwg_sync(zwg_ctx *ctx) {
    if (!ctx) return fail(nullptr, "null context");
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipStreamSynchronize", e);
    return ZWG_OK;
}

int zwg_attention_dev(zwg_ctx *ctx, const float *q, const float *k, const float *v, const zwg_attn_shape *shape,
                      float *out) {
    if (!ctx || !shape) return fail(ctx, "null context or shape");
    const zwg_batch one{1, 0, 0, 0, 0, nullptr};
    return run(ctx, ctx_exec(ctx), q, k, v, *shape, one, out);
}

int zwg_attention_batch_dev(zwg_ctx *ctx, const float *q, const float *k, const float *v,
                            const zwg_attn_shape *shape, const zwg_batch *batch, float *out) {
    if (!ctx || !shape || !batch) return fail(ctx, "null context, shape or batch");
    return run(ctx, ctx_exec(ctx), q, k, v, *shape, *batch, out);
}

int zwg_attention_ex(zwg_ctx *ctx, const float *q, const float *k, const float *v, const zwg_attn_shape *shape,
                     float *out) {
    if (!ctx || !shape) return fail(ctx, "null context or shape");
    const zwg_attn_shape &s = *shape;
    const std::string msg = check_shape(s);
    if (!msg.empty()) return fail(ctx, msg);
    if (s.n_q == 0) return ZWG_OK;
    if (!q || !out || (s.n_kv && (!k || !v))) return fail(ctx, "null tensor pointer");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    const uint64_t F = sizeof(float);
    const uint64_t hd = s.n_head * s.d, kvd = s.n_head_kv * s.d;
    // spans the reference reads: q rows, K rows or KT rows (n_kv columns of the last one), V rows
    const uint64_t q_n = (s.n_q - 1) * s.q_stride + hd;
    const uint64_t k_n = s.n_kv == 0 ? 0 : s.kt_stride ? (kvd - 1) * s.kt_stride + s.n_kv : (s.n_kv - 1) * s.kv_stride + kvd;
    const uint64_t v_n = s.n_kv == 0 ? 0 : (s.n_kv - 1) * s.kv_stride + kvd;
    const uint64_t o_n = (s.n_q - 1) * s.out_stride + hd;
    // +4 floats: a 16-byte key load at the end of the last transposed row stays in the buffer
    if (ensure_stage(ctx, 0, q_n * F) || ensure_stage(ctx, 1, (k_n + 4) * F) || ensure_stage(ctx, 2, (v_n + 4) * F) ||
        ensure_stage(ctx, 3, o_n * F))
        return ZWG_ERROR;
    e = hipMemcpyAsync(ctx->stage[0], q, q_n * F, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && k_n) e = hipMemcpyAsync(ctx->stage[1], k, k_n * F, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && v_n) e = hipMemcpyAsync(ctx->stage[2], v, v_n * F, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipMemcpyAsync (upload)", e);
    const zwg_batch one{1, 0, 0, 0, 0, nullptr};
    Exec x = ctx_exec(ctx);
    // the kernels that write out raise these words to the largest |value| they write (read back
    // with the result)
    x.out_max = ctx->out_max_word;
    e = hipMemsetAsync(ctx->out_max_word, 0, zwg::kOutMaxBytes, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipMemsetAsync (result maximum)", e);
    Plan p;
    int rc = run(ctx, x, ctx->stage[0], ctx->stage[1], ctx->stage[2], s, one, ctx->stage[3], &p);
    if (rc != ZWG_OK) return rc;
    uint32_t slots[zwg::kOutMaxSlots * zwg::kOutMaxStride];
    e = hipMemcpyAsync(slots, ctx->out_max_word, sizeof slots, hipMemcpyDeviceToHost, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipMemcpyAsync (result maximum)", e);
    // copy back only each row's n_head*d columns: out's other columns stay the caller's (waits for
    // the stream, so the maximum has arrived too)
    rc = download_rows(ctx, out, ctx->stage[3], s.n_q, hd, s.out_stride);
    if (rc != ZWG_OK) return rc;
    uint32_t out_max = 0;
    for (int i = 0; i < zwg::kOutMaxSlots; ++i) out_max = std::max(out_max, slots[i * zwg::kOutMaxStride]);
    // The reference gives finite, f32-accurate results for any finite input (src/ops.zig:562-590).
    // The x3 dense kernel meets that when its result is finite and not tiny; otherwise the call is
    // computed again on the fp32-MFMA kernel (which reproduces any NaN or infinity the inputs
    // themselves carry):
    //  - keys (and scaled queries) beyond f16 range make the rows that see them NaN;
    //  - the f16 split of V (and of P) has an absolute error floor near 2^-25 (the spacing of f16
    //    subnormals, where the low terms of values below 2^-3 land): a result whose largest |value|
    //    is below 2^-9 could miss the x3 bar (3e-5 normwise) relative to it.
    constexpr uint32_t kX3SmallResult = 0x3b000000u; // 2^-9
    const bool x3_off_range = out_max >= 0x7f800000u || out_max < kX3SmallResult;
    if (p.kernel == 1 && x.dense_math != ZWG_DENSE_FP32 && x3_off_range) {
        x.out_max = nullptr;
        x.dense_math = ZWG_DENSE_FP32;
        rc = run(ctx, x, ctx->stage[0], ctx->stage[1], ctx->stage[2], s, one, ctx->stage[3]);
        if (rc != ZWG_OK) return rc;
        rc = download_rows(ctx, out, ctx->stage[3], s.n_q, hd, s.out_stride);
        if (rc != ZWG_OK) return rc;
    }
    return ZWG_OK;
}

int zwg_attention(zwg_ctx *ctx, const float *q, const float *k, const float *v, uint64_t n_q, uint64_t n_kv,
                  uint64_t n_state, uint64_t n_head, int causal, float *out) {
    if (n_head == 0) return fail(ctx, "n_head must be positive");
    zwg_attn_shape s{};
    s.n_q = n_q;
    s.n_kv = n_kv;
    s.n_head = n_head;
    s.n_head_kv = n_head;
    s.d = n_state / n_head;
    s.q_stride = n_state;
    s.kv_stride = n_state;
    s.out_stride = n_state;
    s.kt_stride = 0;
    s.causal = causal ? 1u : 0u;
    return zwg_attention_ex(ctx, q, k, v, &s, out);
}

// ---- the allocation-free entry point -------------------------------------------------------
//
// Split partials live in a file-scope device array of this library, one copy per GPU (the code
// object's own global memory, set up when the library's kernels are loaded on that GPU).  In host
// code `scratch` names a host-side stand-in, not device memory: its device address is taken once
// per GPU with hipGetSymbolAddress, with that GPU current, and only that address is passed on.

} // extern "C"

namespace {

constexpr uint64_t kScratchBytes = ZWG_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size");
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxDevices] = {};

// scratch's address on the current device (taken on the first call there)
hipError_t scratch_on_current_device(float **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

} // namespace

extern "C" int zwg_attention_batch_noalloc(const float *q, const float *k, const float *v, const zwg_attn_shape *shape,
                                           const zwg_batch *batch, float *out, uint32_t dense_math,
                                           void *hip_stream) {
    if (!shape) return fail(nullptr, "null shape");
    if (dense_math > ZWG_DENSE_FP32) return fail(nullptr, "unknown dense_math");
    const zwg_batch one{1, 0, 0, 0, 0, nullptr};
    const zwg_batch &b = batch ? *batch : one;
    std::string msg = check_shape(*shape);
    if (msg.empty()) msg = check_batch(*shape, b);
    if (!msg.empty()) return fail(nullptr, msg);
    // the plan of a context with the default workspace; refused here when its partials exceed
    // the static scratch, before the device is touched
    const Plan p = make_plan(*shape, b, kDefaultWorkspace, dense_math);
    if (p.ws_bytes > kScratchBytes) {
        char buf[200];
        snprintf(buf, sizeof buf,
                 "this call's split partials need %llu bytes, more than the %llu-byte static scratch of "
                 "zwg_attention_batch_noalloc (use a context)",
                 (unsigned long long)p.ws_bytes, (unsigned long long)kScratchBytes);
        return fail(nullptr, buf);
    }
    float *ws = nullptr;
    if (p.ws_bytes > 0) {
        const hipError_t e = scratch_on_current_device(&ws);
        if (e != hipSuccess) return fail_hip(nullptr, "hipGetSymbolAddress (static scratch)", e);
    }
    const Exec x{-1, static_cast<hipStream_t>(hip_stream), ws, kScratchBytes, dense_math, kDefaultWorkspace,
                 "the static scratch"};
    return run(nullptr, x, q, k, v, *shape, b, out);
}
