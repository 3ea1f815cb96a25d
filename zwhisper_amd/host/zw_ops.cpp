// C++ mirror of ops.attention / ops.attentionEx (src/ops.zig:545-605) over include/zw_gpu.h.
#include "zw_ops.hpp"

#include <cstdio>
#include <cstdlib>

#include "zw_gpu.h"

namespace zw::ops {
namespace {

[[noreturn]] void panic(const char *what, const char *detail) {
    std::fprintf(stderr, "zwhisper attention: %s%s%s\n", what, detail ? ": " : "", detail ? detail : "");
    std::abort();
}

// One library context per host thread, opened on first use (device from ZW_GPU_DEVICE, else 0)
// and closed at thread exit.
struct ThreadCtx {
    zwg_ctx *ctx = nullptr;
    ~ThreadCtx() {
        if (ctx) zwg_close(ctx);
    }
};
thread_local ThreadCtx t_ctx;

zwg_ctx *context() {
    if (!t_ctx.ctx) {
        const char *env = std::getenv("ZW_GPU_DEVICE");
        const int dev = env ? std::atoi(env) : 0;
        if (zwg_open(dev, nullptr, &t_ctx.ctx) != ZWG_OK) panic("cannot open the GPU", zwg_last_error(nullptr));
    }
    return t_ctx.ctx;
}

} // namespace

std::size_t attentionScratchEx(std::size_t n_q, std::size_t n_kv, std::size_t n_head, std::size_t n_head_kv,
                               std::size_t d) {
    const std::size_t n_kv_pad = (n_kv + V - 1) / V * V;
    const std::size_t n_qblocks = (n_q + q_block - 1) / q_block;
    return n_head_kv * d * n_kv_pad + n_head * n_qblocks * q_block * n_kv_pad;
}

std::size_t attentionScratchKT(std::size_t n_q, std::size_t kt_stride, std::size_t n_head) {
    const std::size_t n_qblocks = (n_q + q_block - 1) / q_block;
    return n_head * n_qblocks * q_block * kt_stride;
}

std::size_t attentionScratch(std::size_t n_q, std::size_t n_kv, std::size_t n_head, std::size_t n_state) {
    return attentionScratchEx(n_q, n_kv, n_head, n_head, n_state / n_head);
}

void attentionEx(Pool *, Slice<const float> q, Slice<const float> k, Slice<const float> v, AttnShape sh,
                 Slice<float>, Slice<float> out) {
    if (sh.n_q == 0) return;
    const std::size_t hd = sh.n_head * sh.d, kvd = sh.n_head_kv * sh.d;
    // the spans the reference indexes (an out-of-range slice panics there in safe builds)
    if (q.len < (sh.n_q - 1) * sh.q_stride + hd) panic("q slice too short", nullptr);
    if (out.len < (sh.n_q - 1) * sh.out_stride + hd) panic("out slice too short", nullptr);
    if (sh.n_kv) {
        const std::size_t k_need =
            sh.kt_stride ? (kvd - 1) * *sh.kt_stride + sh.n_kv : (sh.n_kv - 1) * sh.kv_stride + kvd;
        if (k.len < k_need) panic("k slice too short", nullptr);
        if (v.len < (sh.n_kv - 1) * sh.kv_stride + kvd) panic("v slice too short", nullptr);
    }
    zwg_attn_shape s{};
    s.n_q = sh.n_q;
    s.n_kv = sh.n_kv;
    s.n_head = sh.n_head;
    s.n_head_kv = sh.n_head_kv;
    s.d = sh.d;
    s.q_stride = sh.q_stride;
    s.kv_stride = sh.kv_stride;
    s.out_stride = sh.out_stride;
    s.kt_stride = sh.kt_stride ? *sh.kt_stride : 0;
    s.causal = sh.causal ? 1u : 0u;
    char msg[256];
    if (zwg_check_shape(&s, msg, sizeof msg) != ZWG_OK) panic("precondition", msg);
    zwg_ctx *ctx = context();
    if (zwg_attention_ex(ctx, q.ptr, k.ptr, v.ptr, &s, out.ptr) != ZWG_OK) panic("GPU call failed", zwg_last_error(ctx));
}

void attention(Pool *pool, Slice<const float> q, Slice<const float> k, Slice<const float> v, std::size_t n_q,
               std::size_t n_kv, std::size_t n_state, std::size_t n_head, bool causal, Slice<float> scratch,
               Slice<float> out) {
    attentionEx(pool, q, k, v,
                AttnShape{n_q, n_kv, n_head, n_head, n_state / n_head, n_state, n_state, n_state, causal, std::nullopt},
                scratch, out);
}

} // namespace zw::ops
