// One Whisper encoder layer on the device (include/zw_gpu.h, zwg_encoder_layer_dev): the loop body
// of Encoder.encode (src/encoder.zig:164-175) over a batch of windows held in HBM.
//
//   x_ln = layerNorm(x)                  -> A          (elementwise.hip)
//   q | k | v = x_ln . Wq/Wk/Wv + b      -> B [rows][3 n_state]: three GEMMs writing one
//                                           interleaved buffer, read by attention through its
//                                           q/kv strides (no copies)
//   attn = attention(q, k, v)            -> A          (flash kernel, row-major K, batch = windows)
//   x += attn . Wo + bo                  (residual fused into the GEMM's store)
//   x_ln = layerNorm(x)                  -> A
//   h = gelu(x_ln . W0 + b0)             -> B..C [rows][4 n_state] (GELU fused into the GEMM's store)
//   x += h . W1 + b1                     (residual fused)
//
// Scratch: A (rows n_state) + B (3 rows n_state) + C (rows n_state) floats, the buffers the
// reference allocates per Encoder (src/encoder.zig:98-106), caller-owned as they are.
//
// In the x3 dense mode, for head dims 64 and 128 and windows of a multiple of 4 frames, the K and
// V projections write tile images (kv_image.hpp) instead of f32 rows, and attention copies their
// tiles into LDS as they are: the f16 hi/lo terms it would have formed itself, so the layer's
// results are the same bit for bit, without the attention kernel's K/V loads in f32 and their
// splits.  Scratch then holds A, q [rows][n_state] and the two images (each
// windows x heads x ceil(n_ctx / 32) x 32 x d x 4 bytes, just above rows n_state floats).
#include <hip/hip_runtime.h>

#include <string>

#include "elementwise.hpp"
#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;

extern "C" {

uint64_t zwg_encoder_layer_scratch(uint64_t n_rows, uint64_t n_state) { return 5 * n_rows * n_state; }

int zwg_encoder_layer_dev(zwg_ctx *ctx, float *x, uint64_t n_windows, uint64_t n_ctx, uint64_t n_state,
                          uint64_t n_head, const zwg_enc_layer *w, float *scratch) {
    if (!ctx) return fail(nullptr, "null context");
    if (!x || !w || !scratch) return fail(ctx, "null x, weights or scratch");
    if (n_windows == 0 || n_ctx == 0) return ZWG_OK;
    if (n_head == 0 || n_state % n_head || n_state % 4) return fail(ctx, "n_state must be a multiple of n_head and of 4");
    const uint64_t ns = n_state, rows = n_windows * n_ctx;
    if (rows > 0x7fffffffull) return fail(ctx, "too many rows");
    float *A = scratch, *B = scratch + rows * ns;
    int rc;
    // attention block (src/encoder.zig:164-170)
    if ((rc = zwg_layer_norm_dev(ctx, x, rows, ns, w->attn_ln_w, w->attn_ln_b, 1e-5f, A)) != ZWG_OK) return rc;
    const uint64_t d = ns / n_head, tiles = (n_ctx + 31) / 32;
    const uint64_t img_floats = n_windows * n_head * tiles * 32 * d; // one image, both planes
    if (ctx->dense_math == ZWG_DENSE_X3 && (d == 64 || d == 128) && n_ctx % 4 == 0 &&
        2 * rows * ns + 2 * img_floats <= zwg_encoder_layer_scratch(rows, ns)) {
        float *Q = B, *Kimg = Q + rows * ns, *Vimg = Kimg + img_floats;
        if ((rc = zwg_linear_epi_dev(ctx, A, rows, ns, w->q_w, ZWG_W_F16, w->q_b, ns, Q, ns, ZWG_EPI_NONE)) != ZWG_OK)
            return rc;
        if ((rc = linear_f16_image(ctx, A, rows, ns, w->k_w, nullptr, ns, Kimg, 1, n_ctx, d)) != ZWG_OK) return rc;
        if ((rc = linear_f16_image(ctx, A, rows, ns, w->v_w, w->v_b, ns, Vimg, 2, n_ctx, d)) != ZWG_OK) return rc;
        zwg_attn_shape sh{};
        sh.n_q = n_ctx;
        sh.n_kv = n_ctx;
        sh.n_head = n_head;
        sh.n_head_kv = n_head;
        sh.d = d;
        sh.q_stride = ns;
        sh.kv_stride = ns;
        sh.out_stride = ns;
        sh.causal = 0;
        zwg_batch bt{};
        bt.n_batch = n_windows;
        bt.q_bstride = n_ctx * ns;
        bt.k_bstride = n_ctx * ns;
        bt.v_bstride = n_ctx * ns;
        bt.out_bstride = n_ctx * ns;
        if ((rc = attention_images_dev(ctx, Q, Kimg, Vimg, tiles, sh, bt, A)) != ZWG_OK) return rc;
    } else { // q | k | v rows of B, read by attention through its strides
        if ((rc = zwg_linear_epi_dev(ctx, A, rows, ns, w->q_w, ZWG_W_F16, w->q_b, ns, B, 3 * ns, ZWG_EPI_NONE)) != ZWG_OK)
            return rc;
        if ((rc = zwg_linear_epi_dev(ctx, A, rows, ns, w->k_w, ZWG_W_F16, nullptr, ns, B + ns, 3 * ns, ZWG_EPI_NONE)) !=
            ZWG_OK)
            return rc;
        if ((rc = zwg_linear_epi_dev(ctx, A, rows, ns, w->v_w, ZWG_W_F16, w->v_b, ns, B + 2 * ns, 3 * ns, ZWG_EPI_NONE)) !=
            ZWG_OK)
            return rc;
        zwg_attn_shape sh{};
        sh.n_q = n_ctx;
        sh.n_kv = n_ctx;
        sh.n_head = n_head;
        sh.n_head_kv = n_head;
        sh.d = ns / n_head;
        sh.q_stride = 3 * ns;
        sh.kv_stride = 3 * ns;
        sh.out_stride = ns;
        sh.kt_stride = 0;
        sh.causal = 0;
        zwg_batch bt{};
        bt.n_batch = n_windows;
        bt.q_bstride = n_ctx * 3 * ns;
        bt.k_bstride = n_ctx * 3 * ns;
        bt.v_bstride = n_ctx * 3 * ns;
        bt.out_bstride = n_ctx * ns;
        bt.n_kv_dev = nullptr;
        if ((rc = zwg_attention_batch_dev(ctx, B, B + ns, B + 2 * ns, &sh, &bt, A)) != ZWG_OK) return rc;
    }
    if ((rc = zwg_linear_epi_dev(ctx, A, rows, ns, w->o_w, ZWG_W_F16, w->o_b, ns, x, ns, ZWG_EPI_ADD)) != ZWG_OK)
        return rc;
    // MLP block (src/encoder.zig:172-175)
    if ((rc = zwg_layer_norm_dev(ctx, x, rows, ns, w->mlp_ln_w, w->mlp_ln_b, 1e-5f, A)) != ZWG_OK) return rc;
    if ((rc = zwg_linear_epi_dev(ctx, A, rows, ns, w->mlp0_w, ZWG_W_F16, w->mlp0_b, 4 * ns, B, 4 * ns, ZWG_EPI_GELU)) !=
        ZWG_OK)
        return rc;
    return zwg_linear_epi_dev(ctx, B, rows, 4 * ns, w->mlp1_w, ZWG_W_F16, w->mlp1_b, ns, x, ns, ZWG_EPI_ADD);
}

} // extern "C"
