// The Whisper text decoder on the device (include/zw_gpu.h, zwg_decoder_*): Decoder.setAudio
// (src/decoder.zig:151-159) and Decoder.forward (src/decoder.zig:165-205) for a batch of windows
// decoded in lockstep, one token per window per step, with the caches in HBM as zwg_kv objects.
//
// A step over m windows (X: residual stream, A: normalised rows, Q, T: attention in and out,
// H: MLP hidden rows -- the reference's x, x_ln, q, attn and hidden, src/decoder.zig:57-63):
//
//   X = te.row(tok) + pe[pos]; A = attn_ln(X)        q8p_embed_ln_kernel (one launch)
//   per layer:
//     Q = q(A); k(A), v(A) -> self cache rows at pos  stream + linear_split_sum_qkv_kernel, which
//                                                     also writes the key counts pos + 1
//     T = attention(Q, self cache[0 .. pos])           decode kernel (+ merge)
//     X += o(T); A = cross_ln(X)                       stream + linear_split_sum_add_ln_kernel
//     T = attention(cq(A), cross cache)                stream (partials to P) + decode kernel, whose
//                                                     q load adds the partials and bias (+ merge)
//     X += co(T); A = mlp_ln(X)                        stream + linear_split_sum_add_ln_kernel
//     H = gelu(mlp0(A))                                stream + split sum (GELU in its store)
//     X += mlp1(H); A = next layer's attn_ln(X), or the final ln after the last layer
//   logits = A . te^T                                  stream (unsplit)
//
// 12-14 launches per layer where the same step as separate calls (layer norm, q/k/v projections,
// append, add) takes 19-21.  The fused launches form the same values in the same order as the
// separate ones (the split sums in split order, the add, layer_norm_regs for every norm), so the
// results are equal bit for bit.  The self-attention is the reference's causal call with one
// query, whose only row sees every cached key: it runs as a non-causal call over each window's
// own key count (which lets a window whose position is off the cache, with no keys, through).
#include <hip/hip_runtime.h>

#include <string>

#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;

namespace {

constexpr float kLnEps = 1e-5f; // ops.layerNorm (src/ops.zig:342-344)
// scratch: X, A, Q, T (m rows each), H (4 m rows), P (kMaxQParts m rows: the cross-attention
// query's k-split partials), then the self-attention key counts
constexpr int kMaxQParts = 8; // the decode kernels' load_q takes at most this many

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

// Shapes shared by setAudio and forward: the model's sizes and both caches.
std::string check_decoder(const zwg_ctx *ctx, const zwg_decoder &dec, uint64_t n_seq_needed) {
    const uint64_t ns = dec.n_state, H = dec.n_head;
    if (!dec.layers || dec.n_layer == 0) return "a decoder needs n_layer >= 1 layers";
    if (H == 0 || ns % H) return "n_state must be a multiple of n_head";
    if (ns % 4 || ns <= 256 || ns > 2048) return "n_state must be a multiple of 4, above 256 and at most 2048";
    const uint64_t d = ns / H;
    if (d != 32 && d != 64 && d != 128) return "head dim n_state / n_head must be 32, 64 or 128";
    const zwg_kv *kvs[2] = {dec.self_kv, dec.cross_kv};
    for (int c = 0; c < 2; ++c) {
        const zwg_kv *kv = kvs[c];
        const char *name = c ? "cross cache" : "self cache";
        if (!kv) return std::string("null ") + name;
        if (kv->ctx != ctx) return std::string("the ") + name + " belongs to another context (or its context is closed)";
        const zwg_kv_desc &k = kv->desc;
        if (k.layout != ZWG_KV_ROW || k.n_head_kv != H || k.d != d || k.rope_base != 0.0)
            return std::string("the ") + name + " must be ZWG_KV_ROW with n_head_kv = n_head, d = n_state / n_head and no rotary positions";
        if (k.n_layer < dec.n_layer) return std::string("the ") + name + " has fewer layers than the decoder";
        if (k.n_seq < n_seq_needed) return std::string("windows out of range of the ") + name;
    }
    return "";
}

} // namespace

extern "C" {

int zwg_decoder_set_audio_dev(zwg_ctx *ctx, const zwg_decoder *dec, const float *enc, uint64_t n_windows,
                              uint64_t seq0) {
    if (!ctx) return fail(nullptr, "null context");
    if (!dec) return fail(ctx, "null decoder");
    if (n_windows == 0) return ZWG_OK;
    std::string msg = check_decoder(ctx, *dec, seq0 + n_windows);
    if (!msg.empty()) return fail(ctx, msg);
    const uint64_t ns = dec->n_state;
    for (uint64_t l = 0; l < dec->n_layer && msg.empty(); ++l) {
        const zwg_dec_layer &L = dec->layers[l];
        msg = check_q8(L.ck_w, ns, ns, "ck_w");
        if (msg.empty()) msg = check_q8(L.cv_w, ns, ns, "cv_w");
        if (msg.empty()) msg = check_vec(L.cv_b, false, "cv_b");
    }
    if (!msg.empty()) return fail(ctx, msg);
    if (!enc || !aligned16(enc)) return fail(ctx, "enc must be non-null and 16-byte aligned");
    const zwg_kv *kv = dec->cross_kv;
    const uint64_t rows = n_windows * kv->desc.n_ctx;
    // the windows' cross caches are consecutive (layer, sequence) blocks of n_audio_ctx rows, so one
    // call writes every window's rows (src/decoder.zig:155-156: ops.linear into cross_k / cross_v)
    for (uint64_t l = 0; l < dec->n_layer; ++l) {
        const zwg_dec_layer &L = dec->layers[l];
        const uint64_t at = (l * kv->desc.n_seq + seq0) * kv->per_seq;
        int rc = zwg_linear_q8w_dev(ctx, enc, rows, L.ck_w, nullptr, kv->k + at);
        if (rc == ZWG_OK) rc = zwg_linear_q8w_dev(ctx, enc, rows, L.cv_w, L.cv_b, kv->v + at);
        if (rc != ZWG_OK) return rc;
    }
    return ZWG_OK;
}

uint64_t zwg_decoder_scratch(uint64_t m, uint64_t n_state) {
    return (8 + kMaxQParts) * m * n_state + (m + 3) / 4 * 4;
}

int zwg_decoder_step_dev(zwg_ctx *ctx, const zwg_decoder *dec, const int32_t *tokens, const int32_t *pos, uint64_t m,
                         uint64_t seq0, float *logits, float *scratch) {
    if (!ctx) return fail(nullptr, "null context");
    if (!dec) return fail(ctx, "null decoder");
    if (m == 0) return ZWG_OK;
    if (m > 64) return fail(ctx, "a decoder step takes at most 64 windows");
    std::string msg = check_decoder(ctx, *dec, seq0 + m);
    if (!msg.empty()) return fail(ctx, msg);
    const uint64_t ns = dec->n_state, H = dec->n_head;
    msg = check_q8(dec->te, dec->n_vocab, ns, "te");
    if (msg.empty()) msg = check_vec(dec->pe, true, "pe");
    if (msg.empty()) msg = check_vec(dec->ln_w, true, "ln_w");
    if (msg.empty()) msg = check_vec(dec->ln_b, true, "ln_b");
    for (uint64_t l = 0; l < dec->n_layer && msg.empty(); ++l) {
        const zwg_dec_layer &L = dec->layers[l];
        const zwg_q8w *sq[6] = {L.q_w, L.k_w, L.v_w, L.o_w, L.cq_w, L.co_w};
        const char *sq_names[6] = {"q_w", "k_w", "v_w", "o_w", "cq_w", "co_w"};
        for (int j = 0; j < 6 && msg.empty(); ++j) msg = check_q8(sq[j], ns, ns, sq_names[j]);
        if (msg.empty()) msg = check_q8(L.mlp0_w, 4 * ns, ns, "mlp0_w");
        if (msg.empty()) msg = check_q8(L.mlp1_w, ns, 4 * ns, "mlp1_w");
        const float *norms[6] = {L.attn_ln_w, L.attn_ln_b, L.cross_ln_w, L.cross_ln_b, L.mlp_ln_w, L.mlp_ln_b};
        for (int j = 0; j < 6 && msg.empty(); ++j) msg = check_vec(norms[j], true, "layer norm weights");
        const float *biases[7] = {L.q_b, L.v_b, L.o_b, L.cq_b, L.co_b, L.mlp0_b, L.mlp1_b};
        for (int j = 0; j < 7 && msg.empty(); ++j) msg = check_vec(biases[j], false, "biases");
    }
    if (!msg.empty()) return fail(ctx, msg);
    if (!tokens || !pos) return fail(ctx, "null tokens or pos");
    if (!logits || !scratch || !aligned16(logits) || !aligned16(scratch))
        return fail(ctx, "logits and scratch must be non-null and 16-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);

    float *X = scratch, *A = X + m * ns, *Q = A + m * ns, *T = Q + m * ns, *Hd = T + m * ns, *P = Hd + 4 * m * ns;
    int32_t *n_kv = reinterpret_cast<int32_t *>(P + kMaxQParts * m * ns);
    zwg_kv *self = dec->self_kv, *cross = dec->cross_kv;
    int rc = q8w_embed_ln(ctx, dec->te, tokens, dec->pe, pos, self->desc.n_ctx, m, X, dec->layers[0].attn_ln_w,
                          dec->layers[0].attn_ln_b, kLnEps, A);
    if (rc != ZWG_OK) return rc;

    // one query per window over row-major caches (src/decoder.zig:184, :191)
    zwg_attn_shape sh{};
    sh.n_q = 1;
    sh.n_head = H;
    sh.n_head_kv = H;
    sh.d = ns / H;
    sh.q_stride = ns;
    sh.kv_stride = ns;
    sh.out_stride = ns;
    sh.causal = 0;
    zwg_batch bt{};
    bt.n_batch = m;
    bt.q_bstride = ns;
    bt.out_bstride = ns;

    for (uint64_t l = 0; l < dec->n_layer; ++l) {
        const zwg_dec_layer &L = dec->layers[l];
        // masked self-attention over the cache (src/decoder.zig:178-187)
        const zwg_q8w *qkv[3] = {L.q_w, L.k_w, L.v_w};
        const float *qkv_b[3] = {L.q_b, nullptr, L.v_b};
        if ((rc = linear_q8w_qkv_kv(ctx, A, m, qkv, qkv_b, Q, self, l, seq0, pos, n_kv)) != ZWG_OK) return rc;
        const uint64_t s_at = (l * self->desc.n_seq + seq0) * self->per_seq;
        sh.n_kv = self->desc.n_ctx;
        bt.k_bstride = bt.v_bstride = self->per_seq;
        bt.n_kv_dev = n_kv;
        if ((rc = zwg_attention_batch_dev(ctx, Q, self->k + s_at, self->v + s_at, &sh, &bt, T)) != ZWG_OK) return rc;
        if ((rc = linear_q8w_add_ln(ctx, T, m, L.o_w, L.o_b, X, L.cross_ln_w, L.cross_ln_b, kLnEps, A)) != ZWG_OK)
            return rc;
        // cross-attention over the audio (src/decoder.zig:190-194): the query projection's k-split
        // partials go to P and the attention's q load adds them (and the bias)
        int n_parts = 0;
        if ((rc = linear_q8w_parts(ctx, A, m, L.cq_w, P, kMaxQParts, &n_parts)) != ZWG_OK) return rc;
        const uint64_t c_at = (l * cross->desc.n_seq + seq0) * cross->per_seq;
        sh.n_kv = cross->desc.n_ctx;
        bt.k_bstride = bt.v_bstride = cross->per_seq;
        bt.n_kv_dev = nullptr;
        if ((rc = attention_qparts_dev(ctx, P, n_parts, m * ns, L.cq_b, cross->k + c_at, cross->v + c_at, sh, bt,
                                       T)) != ZWG_OK)
            return rc;
        if ((rc = linear_q8w_add_ln(ctx, T, m, L.co_w, L.co_b, X, L.mlp_ln_w, L.mlp_ln_b, kLnEps, A)) != ZWG_OK)
            return rc;
        // mlp (src/decoder.zig:197-201), then the next block's attn_ln or the final ln (:203)
        if ((rc = zwg_linear_q8w_epi_dev(ctx, A, m, L.mlp0_w, L.mlp0_b, Hd, ZWG_EPI_GELU)) != ZWG_OK) return rc;
        const bool last = l + 1 == dec->n_layer;
        const float *nw = last ? dec->ln_w : dec->layers[l + 1].attn_ln_w;
        const float *nb = last ? dec->ln_b : dec->layers[l + 1].attn_ln_b;
        if ((rc = linear_q8w_add_ln(ctx, Hd, m, L.mlp1_w, L.mlp1_b, X, nw, nb, kLnEps, A)) != ZWG_OK) return rc;
    }
    // logits of every window's token (src/decoder.zig:203-204)
    return zwg_linear_q8w_dev(ctx, A, m, dec->te, nullptr, logits);
}

} // extern "C"
