// Qwen2's decode step on the device (include/zw_gpu.h, zwg_llm_step_dev): Model.forward
// (src/llm.zig:169-216) with one new token in each of m sequences decoded in lockstep, the caches
// in HBM as one zwg_kv (transposed keys, rotary positions).
//
// A step over m sequences (X: residual stream, H: normalised rows, Q, T: attention in and out,
// G, U: MLP gate and up rows -- the reference's x, h, q, attn, gate and up, src/llm.zig:139-146):
//
//   X = embd.row(tok); H = rmsNorm(X, attn_norm)      q8p_embed_ln_kernel (RMS), one launch
//   per layer:
//     Q = rope(q(H)); rope(k(H)) -> K^T cache, v(H) -> V cache at pos
//                                                    stream + linear_split_sum_qkv_kernel, which
//                                                    also writes the key counts pos + 1
//     T = attention(Q, caches[0 .. pos])             decode kernel over transposed keys (+ merge)
//     X += o(T); H = rmsNorm(X, ffn_norm)            stream + linear_split_sum_add_ln_wide_kernel
//                                                    (RMS), which also splits H into f16 hi/lo
//                                                    halves when the gate/up call reads a split x
//     G = silu(gate(H)) * up(H)                      one stream launch over both weight sets, each
//                                                    workgroup on the same columns of both (a
//                                                    SwiGLU pair; + one split sum when k is split);
//                                                    no x split launch of its own
//     X += down(G); H = next layer's attn_norm(X), or the output norm after the last layer
//                                                    stream + the sum, residual add and norm
//   logits = H . output^T                           one stream launch (33..64 sequences: x split by
//                                                    the last down projection's sum kernel)
//
// The fused launches form the same values in the same order as the separate calls (the split
// sums in split order, the residual add, zwg_ew::rms_norm_regs for every norm, the x split's f16
// rounding), so the results are equal bit for bit.  The attention is the reference's causal call with one query, whose only
// row sees every cached key: it runs non-causal over each sequence's own key count.
#include <hip/hip_runtime.h>

#include <string>

#include "elementwise.hpp"
#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

std::string check_q8(const zwg_q8w *w, uint64_t n, uint64_t k, const char *name) {
    uint64_t wn = 0, wk = 0;
    if (!w) return std::string("null weights ") + name;
    if (zwg_q8w_shape(w, &wn, &wk) != ZWG_OK) return std::string("closed weights ") + name;
    if (wn != n || wk != k)
        return std::string("weights ") + name + " are " + std::to_string(wn) + " x " + std::to_string(wk) +
               ", expected " + std::to_string(n) + " x " + std::to_string(k);
    return "";
}

std::string check_vec(const float *p, bool required, const char *name) {
    if (!p) return required ? std::string("null ") + name : "";
    return aligned16(p) ? "" : std::string(name) + " must be 16-byte aligned";
}

std::string check_llm(const zwg_ctx *ctx, const zwg_llm &lm, uint64_t n_seq_needed) {
    const uint64_t ne = lm.n_embd, H = lm.n_head, Hk = lm.n_head_kv;
    if (!lm.layers || lm.n_layer == 0) return "a model needs n_layer >= 1 layers";
    if (lm.reserved) return "reserved must be 0";
    if (H == 0 || Hk == 0 || ne % H || H % Hk) return "n_embd must be a multiple of n_head, n_head of n_head_kv";
    if (ne % 4 || ne <= 256 || ne > 4096) return "n_embd must be a multiple of 4, above 256 and at most 4096";
    if (lm.n_ff == 0 || lm.n_ff % 4) return "n_ff must be a positive multiple of 4";
    if (!(lm.eps >= 0.0f)) return "eps must be >= 0";
    const uint64_t d = ne / H;
    if (d != 32 && d != 64 && d != 128) return "head dim n_embd / n_head must be 32, 64 or 128";
    const zwg_kv *kv = lm.kv;
    if (!kv) return "null cache";
    if (kv->ctx != ctx) return "the cache belongs to another context (or its context is closed)";
    const zwg_kv_desc &k = kv->desc;
    if (k.layout != ZWG_KV_KT || k.n_head_kv != Hk || k.d != d || !(k.rope_base > 0.0))
        return "the cache must be ZWG_KV_KT with the model's n_head_kv, d = n_embd / n_head and rotary positions";
    if (k.n_layer < lm.n_layer) return "the cache has fewer layers than the model";
    if (k.n_seq < n_seq_needed) return "sequences out of range of the cache";
    std::string msg = check_q8(lm.embd, lm.n_vocab, ne, "embd");
    if (msg.empty()) msg = check_q8(lm.output, lm.n_vocab, ne, "output");
    if (msg.empty()) msg = check_vec(lm.output_norm, true, "output_norm");
    const uint64_t kvw = Hk * d;
    for (uint64_t l = 0; l < lm.n_layer && msg.empty(); ++l) {
        const zwg_llm_layer &L = lm.layers[l];
        msg = check_q8(L.wq, ne, ne, "wq");
        if (msg.empty()) msg = check_q8(L.wk, kvw, ne, "wk");
        if (msg.empty()) msg = check_q8(L.wv, kvw, ne, "wv");
        if (msg.empty()) msg = check_q8(L.wo, ne, ne, "wo");
        if (msg.empty()) msg = check_q8(L.w_gate, lm.n_ff, ne, "w_gate");
        if (msg.empty()) msg = check_q8(L.w_up, lm.n_ff, ne, "w_up");
        if (msg.empty()) msg = check_q8(L.w_down, ne, lm.n_ff, "w_down");
        if (msg.empty()) msg = check_vec(L.attn_norm, true, "attn_norm");
        if (msg.empty()) msg = check_vec(L.ffn_norm, true, "ffn_norm");
        const float *biases[3] = {L.bq, L.bk, L.bv};
        for (int j = 0; j < 3 && msg.empty(); ++j) msg = check_vec(biases[j], false, "biases");
    }
    return msg;
}

} // namespace

extern "C" {

uint64_t zwg_llm_scratch(uint64_t m, uint64_t n_embd, uint64_t n_ff) {
    return 4 * m * n_embd + 2 * m * n_ff + (m + 3) / 4 * 4 + q8w_xcvt_halves(n_embd) / 2;
}

int zwg_llm_step_dev(zwg_ctx *ctx, const zwg_llm *lm, const int32_t *tokens, const int32_t *pos, uint64_t m,
                     uint64_t seq0, float *logits, float *scratch) {
    if (!ctx) return fail(nullptr, "null context");
    if (!lm) return fail(ctx, "null model");
    if (m == 0) return ZWG_OK;
    if (m > 64) return fail(ctx, "a decode step takes at most 64 sequences");
    const std::string msg = check_llm(ctx, *lm, seq0 + m);
    if (!msg.empty()) return fail(ctx, msg);
    if (!tokens || !pos) return fail(ctx, "null tokens or pos");
    if (!logits || !scratch || !aligned16(logits) || !aligned16(scratch))
        return fail(ctx, "logits and scratch must be non-null and 16-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);

    const uint64_t ne = lm->n_embd, nff = lm->n_ff, H = lm->n_head, Hk = lm->n_head_kv, d = ne / H;
    const int rms = zwg_ew::kNormRms;
    float *X = scratch, *Hn = X + m * ne, *Q = Hn + m * ne, *T = Q + m * ne, *G = T + m * ne, *U = G + m * nff;
    int32_t *n_kv = reinterpret_cast<int32_t *>(U + m * nff);
    // the ffn-normed rows split for the gate/up call, when that call reads a split pass (written by
    // the o projection's sum kernel, so the call needs no split launch of its own)
    _Float16 *xc = reinterpret_cast<_Float16 *>(reinterpret_cast<float *>(n_kv) + (m + 3) / 4 * 4);
    zwg_kv *kv = lm->kv;
    // src/llm.zig:175: embd.row, then the first block's attn_norm (:178)
    int rc = q8w_embed_ln(ctx, lm->embd, tokens, nullptr, pos, 0, m, X, lm->layers[0].attn_norm, nullptr, lm->eps, Hn,
                          rms);
    if (rc != ZWG_OK) return rc;

    // one query per sequence over its transposed key cache (src/llm.zig:191-202)
    zwg_attn_shape sh{};
    sh.n_q = 1;
    sh.n_kv = kv->desc.n_ctx;
    sh.n_head = H;
    sh.n_head_kv = Hk;
    sh.d = d;
    sh.q_stride = ne;
    sh.kv_stride = Hk * d;
    sh.out_stride = ne;
    sh.kt_stride = kv->desc.n_ctx;
    sh.causal = 0;
    zwg_batch bt{};
    bt.n_batch = m;
    bt.q_bstride = ne;
    bt.k_bstride = kv->per_seq;
    bt.v_bstride = kv->per_seq;
    bt.out_bstride = ne;
    bt.n_kv_dev = n_kv;

    const zwg_q8w *gu0[2] = {lm->layers[0].w_gate, lm->layers[0].w_up};
    _Float16 *gu_xc = q8w_group_reads_xcvt(m, 2, gu0) ? xc : nullptr;
    // likewise the output-normed rows for the logits, from the last down projection's sum kernel
    _Float16 *out_xc = q8w_group_reads_xcvt(m, 1, &lm->output) ? xc : nullptr;
    for (uint64_t l = 0; l < lm->n_layer; ++l) {
        const zwg_llm_layer &L = lm->layers[l];
        // src/llm.zig:179-190: q/k/v, rotary positions, the cache writes
        const zwg_q8w *qkv[3] = {L.wq, L.wk, L.wv};
        const float *qkv_b[3] = {L.bq, L.bk, L.bv};
        if ((rc = linear_q8w_qkv_kv(ctx, Hn, m, qkv, qkv_b, Q, kv, l, seq0, pos, n_kv)) != ZWG_OK) return rc;
        const uint64_t at = (l * kv->desc.n_seq + seq0) * kv->per_seq;
        if ((rc = zwg_attention_batch_dev(ctx, Q, kv->k + at, kv->v + at, &sh, &bt, T)) != ZWG_OK) return rc;
        // :203-204 and the ffn norm (:206)
        if ((rc = linear_q8w_add_ln(ctx, T, m, L.wo, nullptr, X, L.ffn_norm, nullptr, lm->eps, Hn, rms, gu_xc)) !=
            ZWG_OK)
            return rc;
        // :207-211: gate and up, SiLU-gated, down, then the next block's attn_norm or the output
        // norm (:215)
        if ((rc = linear_q8w_swiglu(ctx, Hn, m, L.w_gate, L.w_up, G, gu_xc)) != ZWG_OK) return rc;
        const bool last = l + 1 == lm->n_layer;
        const float *nw = last ? lm->output_norm : lm->layers[l + 1].attn_norm;
        if ((rc = linear_q8w_add_ln(ctx, G, m, L.w_down, nullptr, X, nw, nullptr, lm->eps, Hn, rms,
                                    last ? out_xc : nullptr)) != ZWG_OK)
            return rc;
    }
    // the logits of every sequence's token (src/llm.zig:216)
    float *outs[1] = {logits};
    return linear_q8w_group_xcvt(ctx, Hn, m, 1, &lm->output, nullptr, outs, out_xc);
}

uint64_t zwg_llm_forward_scratch(uint64_t n, uint64_t n_embd, uint64_t n_ff) {
    return n * (6 * n_embd + 2 * n_ff);
}

// Model.forward (src/llm.zig:169-216) over n tokens of one sequence at positions pos0 .. pos0 +
// n - 1: the reference's prompt batch (Model.prompt feeds a prompt in such batches,
// src/llm.zig:258-266), each step the library call of the reference's op: rmsNorm, the q/k/v
// projections (one grouped call), the rotary cache append (q rotated in place), attentionEx over
// the pos0 + n cached keys (causal, transposed keys), o with the residual add in its store, the
// gate/up projections, siluMul, down with the add; then the output norm and the logits of the
// last row only (:214-216).
int zwg_llm_forward_dev(zwg_ctx *ctx, const zwg_llm *lm, const int32_t *tokens, uint64_t n, uint64_t seq,
                        uint64_t pos0, float *logits, float *scratch) {
    if (!ctx) return fail(nullptr, "null context");
    if (!lm) return fail(ctx, "null model");
    if (n == 0) return ZWG_OK;
    const std::string msg = check_llm(ctx, *lm, seq + 1);
    if (!msg.empty()) return fail(ctx, msg);
    if (pos0 + n > lm->kv->desc.n_ctx || n > 0x7fffffffull) return fail(ctx, "pos0 + n is past the cache (n_ctx)");
    if (!tokens) return fail(ctx, "null tokens");
    if (!logits || !scratch || !aligned16(logits) || !aligned16(scratch))
        return fail(ctx, "logits and scratch must be non-null and 16-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);

    const uint64_t ne = lm->n_embd, nff = lm->n_ff, H = lm->n_head, Hk = lm->n_head_kv, d = ne / H;
    const int rms = zwg_ew::kNormRms;
    float *X = scratch, *Hn = X + n * ne, *Q = Hn + n * ne, *T = Q + n * ne, *Kb = T + n * ne, *Vb = Kb + n * ne,
          *G = Vb + n * ne, *U = G + n * nff;
    zwg_kv *kv = lm->kv;
    // :175 and the first block's attn_norm (:178)
    int rc = q8w_embed_ln(ctx, lm->embd, tokens, nullptr, nullptr, 0, n, X, lm->layers[0].attn_norm, nullptr,
                          lm->eps, Hn, rms);
    if (rc != ZWG_OK) return rc;
    zwg_attn_shape sh{};
    sh.n_q = n;
    sh.n_kv = pos0 + n;
    sh.n_head = H;
    sh.n_head_kv = Hk;
    sh.d = d;
    sh.q_stride = ne;
    sh.kv_stride = Hk * d;
    sh.out_stride = ne;
    sh.kt_stride = kv->desc.n_ctx;
    sh.causal = 1;
    // batches the int8 calls stream (at most q8w_stream_rows() rows) take the fused launches of the
    // decode step: the q/k/v projections writing the cache, and the residual projections' split
    // sums adding into x and normalising it for the next block, with the same results
    const bool fused = n <= q8w_stream_rows();
    for (uint64_t l = 0; l < lm->n_layer; ++l) {
        const zwg_llm_layer &L = lm->layers[l];
        if (l > 0 && !fused && (rc = rms_norm(ctx, X, n, ne, L.attn_norm, lm->eps, Hn)) != ZWG_OK) return rc;
        // :179-190
        const zwg_q8w *qkv[3] = {L.wq, L.wk, L.wv};
        const float *qkv_b[3] = {L.bq, L.bk, L.bv};
        float *qkv_out[3] = {Q, Kb, Vb};
        if (fused) {
            if ((rc = linear_q8w_qkv_kv(ctx, Hn, n, qkv, qkv_b, Q, kv, l, seq, nullptr, nullptr, (int64_t)pos0)) !=
                ZWG_OK)
                return rc;
        } else {
            if ((rc = zwg_linear_q8w_group_dev(ctx, Hn, n, 3, qkv, qkv_b, qkv_out)) != ZWG_OK) return rc;
            if ((rc = zwg_kv_append(kv, l, seq, pos0, n, Kb, Vb, Q, H, ne, 0)) != ZWG_OK) return rc;
        }
        // :191-202
        const uint64_t at = (l * kv->desc.n_seq + seq) * kv->per_seq;
        if ((rc = zwg_attention_dev(ctx, Q, kv->k + at, kv->v + at, &sh, T)) != ZWG_OK) return rc;
        // :203-211
        if (fused) {
            if ((rc = linear_q8w_add_ln(ctx, T, n, L.wo, nullptr, X, L.ffn_norm, nullptr, lm->eps, Hn, rms)) != ZWG_OK)
                return rc;
        } else {
            if ((rc = zwg_linear_q8w_epi_dev(ctx, T, n, L.wo, nullptr, X, ZWG_EPI_ADD)) != ZWG_OK) return rc;
            if ((rc = rms_norm(ctx, X, n, ne, L.ffn_norm, lm->eps, Hn)) != ZWG_OK) return rc;
        }
        if (fused) {
            if ((rc = linear_q8w_swiglu(ctx, Hn, n, L.w_gate, L.w_up, G)) != ZWG_OK) return rc;
        } else {
            const zwg_q8w *gu[2] = {L.w_gate, L.w_up};
            float *gu_out[2] = {G, U};
            if ((rc = zwg_linear_q8w_group_dev(ctx, Hn, n, 2, gu, nullptr, gu_out)) != ZWG_OK) return rc;
            if ((rc = zwg_silu_mul_dev(ctx, G, U, n * nff)) != ZWG_OK) return rc;
        }
        if (fused) {
            // the next block's attn_norm, or the output norm (of every row; the logits take the last)
            const float *nw = l + 1 == lm->n_layer ? lm->output_norm : lm->layers[l + 1].attn_norm;
            if ((rc = linear_q8w_add_ln(ctx, G, n, L.w_down, nullptr, X, nw, nullptr, lm->eps, Hn, rms)) != ZWG_OK)
                return rc;
        } else if ((rc = zwg_linear_q8w_epi_dev(ctx, G, n, L.w_down, nullptr, X, ZWG_EPI_ADD)) != ZWG_OK) {
            return rc;
        }
    }
    // :214-216: the last row's output norm and logits
    if (!fused && (rc = rms_norm(ctx, X + (n - 1) * ne, 1, ne, lm->output_norm, lm->eps, Hn + (n - 1) * ne)) != ZWG_OK)
        return rc;
    return zwg_linear_q8w_dev(ctx, Hn + (n - 1) * ne, 1, lm->output, nullptr, logits);
}

} // extern "C"
