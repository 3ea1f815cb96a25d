// The library context behind the opaque zwg_ctx of include/zw_gpu.h, and the error / staging
// helpers the C ABI translation units share (zw_gpu.hip, kv_cache.hip, linear.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "zw_gpu.h"

// An object made from a context (a zwg_kv, a zwg_q8w) that holds device memory of its own.
// zwg_close detaches the ones still alive: `detach` frees their device memory and clears their
// context pointer, so a later destroy only frees the host struct and other calls fail cleanly.
struct ZwgChild {
    void *obj;
    void (*detach)(void *obj);
};

struct zwg_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // recorded on the old stream and waited on by the new one whenever zwg_set_stream switches
    // streams: every call shares the workspace, so work queued on one stream must finish before
    // work on the next touches it
    hipEvent_t switch_event = nullptr;
    float *workspace = nullptr;
    // device words the kernels raise to the largest |out| they write (host drop-in only;
    // zwg::kOutMaxSlots slots 128 bytes apart)
    uint32_t *out_max_word = nullptr;
    uint32_t dense_math = ZWG_DENSE_X3; // products of the dense kernel (zwg_set_dense_math)
    uint64_t workspace_bytes = 0;
    // device staging: q, k, v, out of the host-pointer calls (0-3), and the zero-padded q, k, v, out
    // of calls whose head dim has no kernels of its own (4-7)
    float *stage[8] = {};
    uint64_t stage_bytes[8] = {};
    // pinned host staging for results whose rows are not contiguous in the caller's buffer
    float *host_stage = nullptr;
    uint64_t host_stage_bytes = 0;
    // zwg_limits.staging_bytes was set: every staging buffer was allocated at zwg_open and a call
    // that needs more is refused instead of growing it
    bool fixed_staging = false;
    std::vector<ZwgChild> children;
    std::string err;
};

// A device-resident KV cache (zwg_kv_create, kv_cache.hip); the q/k/v projections with the cache
// append fused into their final store (linear.hip) write into it too.
struct zwg_kv {
    zwg_ctx *ctx = nullptr;
    zwg_kv_desc desc{};
    uint64_t kvw = 0;     // n_head_kv * d
    uint64_t per_seq = 0; // floats of one (layer, sequence) K or V cache: n_ctx * kvw
    float *k = nullptr;   // [layer][sequence][per_seq]
    float *v = nullptr;
    float *cos = nullptr; // [n_ctx][d/2] rotary tables when rope_base > 0
    float *sin = nullptr;
};

namespace zwg_host {

// Record `msg` as the last error (of ctx, and of this thread) and return ZWG_ERROR.
int fail(zwg_ctx *ctx, const std::string &msg);
int fail_hip(zwg_ctx *ctx, const char *what, hipError_t e);
// Grow staging buffer i of ctx to at least `bytes` (synchronises the stream when it grows).
int ensure_stage(zwg_ctx *ctx, int i, uint64_t bytes);
// Copy n_rows rows of `cols` floats, `stride` floats apart, from device `src` to host `dst` (same
// layout; the gaps of dst are left alone), queued on ctx's stream and waited for: one copy when
// the rows are contiguous, else one copy of the whole span into pinned staging and row copies on
// the host.
int download_rows(zwg_ctx *ctx, float *dst, const float *src, uint64_t n_rows, uint64_t cols, uint64_t stride);
// The encoder layer's K/V path (kv_image.hpp): the f16 linear layer writing K (kind 1) or V
// (kind 2) tile images in place of f32 rows -- rows = items * n_ctx (n_ctx % 4 == 0), n = heads * d
// (d 64 or 128) -- and the dense x3 attention reading them (q, out and the shape as for
// zwg_attention_batch_dev, row-major K; img_tiles = ceil(n_kv / 32)).
int linear_f16_image(zwg_ctx *ctx, const float *x, uint64_t rows, uint64_t k, const void *w, const float *bias,
                     uint64_t n, void *img, int kind, uint64_t n_ctx, uint64_t d);
int attention_images_dev(zwg_ctx *ctx, const float *q, const void *k_img, const void *v_img, uint64_t img_tiles,
                         const zwg_attn_shape &s, const zwg_batch &b, float *out);
// zwg_attention_batch_dev whose queries are the n_parts k-split partial sums of their projection
// (part_stride floats apart) plus q_bias: the decode kernels add them in their q load.
int attention_qparts_dev(zwg_ctx *ctx, const float *q_parts, int n_parts, uint64_t part_stride, const float *q_bias,
                         const float *k, const float *v, const zwg_attn_shape &s, const zwg_batch &b, float *out);
// A decode step's projection (m <= 64, k above 256) with its k-split partial sums left in
// parts[n_split][m][n] (parts holds max_parts * m * n floats) and no split-sum launch; the
// split count (2 .. max_parts) goes to *n_split.
int linear_q8w_parts(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, float *parts, int max_parts,
                     int *n_split);
// zwg_linear_q8w_qkv_kv_dev with, when n_kv_out is set, each sequence's key count after the
// append (pos + 1, 0 for a position off the cache) written to n_kv_out[m] by the same launch.
// pos_dev nullptr: the m rows are one sequence's (seq0) tokens at pos0 .. pos0 + m - 1 (a prompt
// batch, m <= q8w_stream_rows()).
int linear_q8w_qkv_kv(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *const *w, const float *const *bias,
                      float *q_out, zwg_kv *kv, uint64_t layer, uint64_t seq0, const int32_t *pos_dev,
                      int32_t *n_kv_out, int64_t pos0 = -1);
// rows up to which the int8 calls stream the resident weights (and the fused calls take)
uint64_t q8w_stream_rows();
// out = silu(x . gate^T) * (x . up^T), m <= q8w_stream_rows() (one stream launch over both sets);
// xcvt_in as for linear_q8w_group_xcvt
int linear_q8w_swiglu(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *gate, const zwg_q8w *up, float *out,
                      const _Float16 *xcvt_in = nullptr);
// A decode step's residual projection and the next norm: x += xin . W^T + bias, then ln_out =
// the norm of x (norm 0: layer norm, 1: RMS norm; m <= q8w_stream_rows(), n <= 4096; linear.hip).  xcvt_out
// (33..64 rows): ln_out also split into f16 hi/lo halves for the next call (q8w_xcvt_halves(n)
// halves), passed to it as xcvt_in.
int linear_q8w_add_ln(zwg_ctx *ctx, const float *xin, uint64_t m, const zwg_q8w *w, const float *bias, float *x,
                      const float *ln_w, const float *ln_b, float eps, float *ln_out, int norm = 0,
                      _Float16 *xcvt_out = nullptr);
uint64_t q8w_xcvt_halves(uint64_t k);
// whether a token-step group call of these weights over m rows streams its x from a split pass
// (and so takes linear_q8w_group_xcvt's xcvt_in)
bool q8w_group_reads_xcvt(uint64_t m, uint32_t n_w, const zwg_q8w *const *w);
// zwg_linear_q8w_group_dev over rows whose split was written by linear_q8w_add_ln (xcvt_in)
int linear_q8w_group_xcvt(zwg_ctx *ctx, const float *x, uint64_t m, uint32_t n_w, const zwg_q8w *const *w,
                          const float *const *bias, float *const *out, const _Float16 *xcvt_in);
// Token embeddings from packed int8 rows plus positional rows (pe may be null), and their norm:
// x[i] = te.row(tok[i]) + pe[pos[i]], ln_out[i] = the norm of x[i] (n <= 4096; linear.hip).
int q8w_embed_ln(zwg_ctx *ctx, const zwg_q8w *te, const int32_t *tok, const float *pe, const int32_t *pos,
                 uint64_t pe_rows, uint64_t m, float *x, const float *ln_w, const float *ln_b, float eps,
                 float *ln_out, int norm = 0);
// Register / unregister an object made from ctx (see ZwgChild).
void add_child(zwg_ctx *ctx, void *obj, void (*detach)(void *));
void remove_child(zwg_ctx *ctx, void *obj);

} // namespace zwg_host
