/*
 * zw_gpu.h — C ABI of the MI355X (gfx950) attention library for zwhisper.
 *
 * It replaces the bodies of zwhisper's `ops.attentionEx` (src/ops.zig:562-590) and
 * `ops.attention` (src/ops.zig:593-605).  Those Zig functions keep their signatures; their
 * bodies call the entry points below through a small Zig binding of this header.
 * The whisper C ABI (include/zwhisper.h) is untouched: attention is internal to it.
 *
 * Conventions (those of include/zwhisper.h:34-42):
 *   - every function returning int gives ZWG_OK (0) on success, ZWG_ERROR (2) on failure;
 *     zwg_last_error() then says why.  No C++ exception crosses this boundary.
 *   - the caller owns every buffer it passes; a context owns its stream and device workspace
 *     and frees them in zwg_close().
 *   - one context per host thread; calls on one context are not thread-safe
 *     (as the zw_* handles, src/capi.zig:3-4).
 *
 * Arithmetic and tolerances (against the f64 closed form of the reference's attention):
 *   - decode (split-K streaming) kernel: f32 FMA.  Bar: max abs 2e-4, normwise relative 1e-3
 *     (||gpu - ref||_inf / ||ref||_inf), the reference's f32 bar; measured ~1e-7.
 *   - dense (encoder / prefill) kernel, ZWG_DENSE_X3 (the default, below): f32 operands split into
 *     f16 hi + lo terms (22 significand bits), three f16 MFMA products per product, f32
 *     accumulation.  Its own bar on N(0,1) inputs: max abs 5e-5 and normwise relative 3e-5
 *     (measured at most 8.4e-7 abs and 1.3e-6 relative on the Whisper / Qwen2 workloads); with scores spread
 *     36x wider it measures 4.5e-5, inside the f32 bar.
 *   - dense kernel, ZWG_DENSE_FP32: fp32 MFMA (v_mfma_f32_32x32x2_f32) throughout; the f32 bar.
 * The absolute bars are for values of order one: an output row is a weighted mean of value rows,
 * so with values up to M in magnitude they scale by M.
 */
#ifndef ZW_GPU_H
#define ZW_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZWG_OK 0
#define ZWG_ERROR 2
#define ZWG_VERSION 2

typedef struct zwg_ctx zwg_ctx;

/*
 * Mirror of ops.AttnShape (src/ops.zig:477-492), field for field.  Query head h reads key/value
 * head h / (n_head / n_head_kv).  Strides are in floats.  kt_stride == 0 stands for Zig's
 * `null`: k is row-major [n_kv][kv_stride] like v.  kt_stride > 0: k is transposed,
 * [n_head_kv][d][kt_stride] (keys along the last axis, as the LLM's cache, src/llm.zig:27).
 * causal: query i sees keys j <= n_kv - n_q + i (src/ops.zig:466), so n_kv >= n_q is required.
 *
 * Limits of this build (checked; ZWG_ERROR otherwise): d a multiple of 4 up to 1024 (the
 * reference takes any d % V == 0, V = 8 or 16); q_stride, kv_stride, out_stride and kt_stride
 * multiples of 4; q, k, v, out 16-byte aligned; n_q, n_kv and n_head below 2^30; n_head * n_batch
 * below 2^31.  The MFMA and split-K kernels are built for d = 32, 64 and 128; any other d up to
 * 128 runs on the kernels of the next of them over zero-padded copies of q, k, v and out that the
 * context keeps (one more read and write of each tensor per call; same results up to f32
 * rounding); d above 128 runs on a plain f32 kernel, one wavefront per query row, unsplit (no
 * model zwhisper runs has such a head dim: it keeps the drop-in whole, untuned).
 * Device buffers: with kt_stride, the last transposed row is read in 16-byte groups, so k must
 * hold (n_head_kv*d - 1)*kt_stride + round_up(n_kv, 4) floats -- no more than the reference
 * itself reads (round_up(n_kv, V) columns of every row, src/ops.zig:529-530).
 */
typedef struct zwg_attn_shape {
    uint64_t n_q;
    uint64_t n_kv;
    uint64_t n_head;
    uint64_t n_head_kv;
    uint64_t d;
    uint64_t q_stride;
    uint64_t kv_stride;
    uint64_t out_stride;
    uint64_t kt_stride;
    uint32_t causal;
    uint32_t reserved; /* must be 0 */
} zwg_attn_shape;

/*
 * A batch of independent attention problems of one shape, laid out at fixed strides (in floats)
 * from the base pointers: item b uses q + b*q_bstride, k + b*k_bstride, v + b*v_bstride,
 * out + b*out_bstride.  n_kv_dev, if not NULL, is a device array of n_batch int32 key counts
 * (each 0 <= n_kv_dev[b] <= shape.n_kv, the capacity): per-item cache lengths, as the decoder
 * windows or LLM sequences of one step have.  Causal items need n_kv_dev[b] >= n_q.
 */
typedef struct zwg_batch {
    uint64_t n_batch;
    uint64_t q_bstride;
    uint64_t k_bstride;
    uint64_t v_bstride;
    uint64_t out_bstride;
    const int32_t *n_kv_dev;
} zwg_batch;

/*
 * Arithmetic of the dense (encoder / prefill) attention kernel (tolerances at the top of this
 * file):
 *   ZWG_DENSE_X3 (default): every product as three f16 MFMA products of operands split into
 *     hi + lo terms (22 significand bits, so a score's error does not grow with large logits),
 *     f32 accumulation, about 2.5x the fp32 kernel's rate.  Keys and values must stay below 65504
 *     in magnitude (f16 range): a larger key gives NaN in the rows that see it, a larger value NaN
 *     in its own output column (head, dimension) of the rows whose 32-row group loads its 32-key
 *     tile -- never a silently wrong finite result
 *     (zwg_attention_ex then recomputes the call in ZWG_DENSE_FP32).  Small values: the split's
 *     low terms of values below 2^-3 are f16 subnormals, so the error has an absolute floor near
 *     2^-25 rather than staying relative; results whose largest |value| is below 2^-9 can miss
 *     the x3 relative bar (zwg_attention_ex recomputes those in ZWG_DENSE_FP32 too).
 *   ZWG_DENSE_FP32: fp32 MFMA (v_mfma_f32_32x32x2_f32) throughout, no range condition.
 * The decode kernels are f32 FMA in either mode.
 */
#define ZWG_DENSE_X3 0u
#define ZWG_DENSE_FP32 1u

/* Sizes and modes fixed when a context opens.  Zero fields take the defaults. */
typedef struct zwg_limits {
    uint64_t workspace_bytes; /* device memory for split partial results (attention key splits,
                                 linear k splits); default 256 MiB */
    uint32_t dense_math;      /* ZWG_DENSE_X3 (0, default) or ZWG_DENSE_FP32 */
    uint32_t reserved;        /* must be 0 */
    uint64_t staging_bytes;   /* bytes of each staging buffer: the host-pointer calls' device copies
                                 of q, k, v and out, the zero-padded copies of calls whose head dim
                                 has no kernel of its own, and the pinned host copy of results with
                                 gaps between rows.  Non-zero: all are allocated here, like the
                                 reference's scratch sized at load (src/ops.zig:545-560), and a call
                                 that would need more is refused, so no call allocates.  0 (default):
                                 each grows on the first call that needs more (that call allocates
                                 and waits for the context's stream). */
} zwg_limits;

/* How a call will run (zwg_plan): which kernel, how the keys are split. */
typedef struct zwg_plan_info {
    uint32_t kernel;        /* 1 = dense MFMA flash kernel, 2 = split-K streaming decode kernel,
                               3 = f32 kernel for head dims above 128 */
    uint32_t rows_per_unit; /* query rows one work unit covers (q-block, or heads x queries) */
    uint64_t chunk_len;     /* keys per split (a multiple of the kernel's key tile) */
    uint64_t max_chunks;    /* splits of the longest row; 1 = no combine pass */
    uint64_t grid_blocks;   /* workgroups launched by the main kernel */
    uint64_t workspace_bytes; /* partial results the call writes (0 when max_chunks == 1) */
} zwg_plan_info;

/* Open a context on HIP device `device` (limits may be NULL).  *out is NULL on failure. */
int zwg_open(int device, const zwg_limits *limits, zwg_ctx **out);
void zwg_close(zwg_ctx *ctx);

/* Why the last call on ctx failed; with ctx == NULL, the last failure on this thread. */
const char *zwg_last_error(const zwg_ctx *ctx);

/* Queue the context's work on a caller's hipStream_t (NULL is HIP's null stream) / the stream
 * in use.  A context starts on a stream of its own; zwg_get_stream right after zwg_open
 * returns it, to switch back later.  Every call of a context uses the same workspace, so a
 * switch orders the new stream after the work already queued on the old one (an event recorded
 * on the old stream, waited on by the new); calls issued on one stream run in issue order.
 * The old stream must still exist at the switch (the event is recorded on it): switch the
 * context away from a caller's stream before destroying that stream, as for any HIP call, a
 * call that names a destroyed stream is undefined. */
int zwg_set_stream(zwg_ctx *ctx, void *hip_stream);
void *zwg_get_stream(const zwg_ctx *ctx);
/* Wait for all work queued on the context's stream. */
int zwg_sync(zwg_ctx *ctx);
/* Switch the dense kernel's arithmetic (ZWG_DENSE_X3 or ZWG_DENSE_FP32) for later calls. */
int zwg_set_dense_math(zwg_ctx *ctx, uint32_t mode);

/*
 * Drop-in for ops.attentionEx (src/ops.zig:562): host pointers, synchronous — `out` holds the
 * result on return, and only each query row's n_head*d columns are written, as in the
 * reference.  Stages q/k/v through device buffers the context keeps (grown on first need, or
 * fixed at zwg_open: zwg_limits.staging_bytes).  It keeps the reference's contract for any
 * finite input: the kernels record the largest |value| they write on the device, and when the
 * x3 dense kernel's result holds a non-finite value (a key, value or scaled query beyond f16
 * range) or is smaller than 2^-9 throughout (below the x3 error floor's reach), the call is
 * computed again on the fp32-MFMA kernel, which has neither condition.
 */
int zwg_attention_ex(zwg_ctx *ctx, const float *q, const float *k, const float *v, const zwg_attn_shape *shape,
                     float *out);

/* Drop-in for ops.attention (src/ops.zig:593): n_head_kv = n_head, d = n_state / n_head,
 * all strides n_state, row-major K. */
int zwg_attention(zwg_ctx *ctx, const float *q, const float *k, const float *v, uint64_t n_q, uint64_t n_kv,
                  uint64_t n_state, uint64_t n_head, int causal, float *out);

/* Device pointers (inputs already in HBM): queued on the context's stream, asynchronous.  In
 * ZWG_DENSE_X3 mode dense calls need |k| < 65504, |v| < 65504 and |q| / sqrt(d) * log2(e) < 65504
 * (rows that meet a larger value come out NaN); ZWG_DENSE_FP32 mode has no such condition. */
int zwg_attention_dev(zwg_ctx *ctx, const float *q, const float *k, const float *v, const zwg_attn_shape *shape,
                      float *out);

/* A batch of problems (see zwg_batch), device pointers, asynchronous. */
int zwg_attention_batch_dev(zwg_ctx *ctx, const float *q, const float *k, const float *v,
                            const zwg_attn_shape *shape, const zwg_batch *batch, float *out);

/*
 * zwg_attention_batch_dev without a context and without any device allocation.  No counterpart in
 * the reference; it is for callers that cannot call hipMalloc -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation.  It runs on the calling thread's current
 * device and on `hip_stream` (NULL: the null stream), with the dense arithmetic `dense_math`, and
 * plans and computes exactly as a context opened with the default workspace (same kernels, same
 * key splits, same results).  batch may be NULL (one item).
 * Split partial results go to a static device array of ZWG_NOALLOC_SCRATCH_BYTES per GPU, which
 * the library holds until the process ends: a call whose partials would need more is refused
 * with an error (zwg_last_error(NULL)) before touching the device.  Nothing in it needs clearing
 * between calls (every partial a merge reads is written by the same call first).  All calls on
 * one GPU share that array: calls that overlap in time on one GPU (different streams, or threads)
 * race on it and give wrong results; calls on one stream run in order and are safe.  Head dims
 * up to 128 other than 32, 64 and 128 need the padded copies of a context and are refused here.
 */
#define ZWG_NOALLOC_SCRATCH_BYTES (64ull << 20)
int zwg_attention_batch_noalloc(const float *q, const float *k, const float *v, const zwg_attn_shape *shape,
                                const zwg_batch *batch, float *out, uint32_t dense_math, void *hip_stream);

/*
 * The plan a call with this shape and batch (NULL = one item) would use, for a context opened
 * with `workspace_bytes` of workspace (0 = default) in the default dense mode (ZWG_DENSE_X3;
 * ZWG_DENSE_FP32 splits causal calls into more chunks).  Host-only: needs no device.
 */
int zwg_plan(const zwg_attn_shape *shape, const zwg_batch *batch, uint64_t workspace_bytes, zwg_plan_info *out);

/* Shape check alone (same rules as the calls), host-only.  0 ok, 2 with a message. */
int zwg_check_shape(const zwg_attn_shape *shape, char *msg, size_t msg_len);

/*
 * Device-resident KV caches.  The reference's callers own host caches and fill them on the
 * CPU: the Whisper decoder writes each token's K/V projections into row-major caches
 * (src/decoder.zig:39-42, :182-183) and a window's cross K/V once (src/decoder.zig:151-159);
 * Qwen2 rotates q and k (NeoX rotary positions, src/llm.zig:182-183, :221-238, tables
 * :128-137), scatters k into a transposed cache and copies v (src/llm.zig:185-190).
 * A zwg_kv keeps those caches in HBM, one per (layer, sequence), and appends to them on the
 * device; attention then reads them in place through zwg_attention_dev / _batch_dev with the
 * pointers and strides of zwg_kv_get_info.  These calls replace the cache writes around
 * ops.attentionEx; the attention entry points above are unchanged.
 */
typedef struct zwg_kv zwg_kv;

#define ZWG_KV_ROW 0u /* k, v: [n_ctx][n_head_kv*d] (Whisper decoder self and cross caches) */
#define ZWG_KV_KT 1u  /* k: [n_head_kv][d][n_ctx] transposed, v: [n_ctx][n_head_kv*d] (Qwen2) */

typedef struct zwg_kv_desc {
    uint64_t n_layer;
    uint64_t n_seq;     /* independent sequences: decoder windows, LLM sequences */
    uint64_t n_ctx;     /* positions per sequence (a multiple of 4 for ZWG_KV_KT) */
    uint64_t n_head_kv;
    uint64_t d;         /* 32, 64 or 128 */
    uint32_t layout;    /* ZWG_KV_ROW or ZWG_KV_KT */
    uint32_t reserved;  /* must be 0 */
    double rope_base;   /* > 0: NeoX rotary positions with this base (qwen2.rope.freq_base,
                           src/llm.zig:101) applied to appended keys and to q; 0: none */
} zwg_kv_desc;

/* Where the caches are, for the attention calls.  Layer l, sequence s: k + l*layer_stride +
 * s*seq_stride (likewise v); a batch of consecutive sequences is a zwg_batch with
 * k_bstride = v_bstride = seq_stride. */
typedef struct zwg_kv_info {
    float *k;
    float *v;
    uint64_t layer_stride; /* floats */
    uint64_t seq_stride;   /* floats */
    uint64_t kv_stride;    /* the attention shape's kv_stride: n_head_kv * d */
    uint64_t kt_stride;    /* the attention shape's kt_stride: n_ctx for ZWG_KV_KT, 0 for ZWG_KV_ROW */
} zwg_kv_info;

/* Flag of zwg_kv_append: k_rows, v_rows (and q) are host memory.  The call stages them through
 * the context, hands the rotated q back, and returns when the cache holds the rows. */
#define ZWG_ROWS_ON_HOST 1u

/* Allocate the caches of `desc` on ctx's device (zeroed; rotary tables built on the host in
 * f64 and rounded to f32, as src/llm.zig:128-137).  *out is NULL on failure.  zwg_close of the
 * context frees the caches of a zwg_kv not destroyed yet; the zwg_kv itself then only accepts
 * zwg_kv_destroy (other calls fail). */
int zwg_kv_create(zwg_ctx *ctx, const zwg_kv_desc *desc, zwg_kv **out);
void zwg_kv_destroy(zwg_kv *kv);
int zwg_kv_get_info(const zwg_kv *kv, zwg_kv_info *out);

/*
 * Append n rows to (layer, seq) at positions pos .. pos+n-1 (pos + n <= n_ctx).  k_rows, v_rows:
 * [n][n_head_kv*d], the new keys and values before rotation.  With rope_base > 0 the keys are
 * rotated at their positions, and q (if not NULL: [n][q_stride], n_head heads of d, rotated in
 * place) too -- src/llm.zig:182-190 as one kernel.  Device pointers (16-byte aligned; q_stride a
 * multiple of 4) and asynchronous on the context's stream, unless flags has ZWG_ROWS_ON_HOST.
 */
int zwg_kv_append(zwg_kv *kv, uint64_t layer, uint64_t seq, uint64_t pos, uint64_t n, const float *k_rows,
                  const float *v_rows, float *q, uint64_t n_head, uint64_t q_stride, uint32_t flags);

/* One new row for each of the sequences seq0 .. seq0+n_seq-1 (a batched decode step), at the
 * positions in the device int32 array pos_dev[n_seq]; row i of k_rows, v_rows and q belongs to
 * sequence seq0 + i.  A position outside [0, n_ctx) is skipped.  Device pointers, asynchronous. */
int zwg_kv_append_batch(zwg_kv *kv, uint64_t layer, uint64_t seq0, uint64_t n_seq, const int32_t *pos_dev,
                        const float *k_rows, const float *v_rows, float *q, uint64_t n_head, uint64_t q_stride);

/* Copy one (layer, seq) cache to host memory (k_host, v_host: n_ctx*n_head_kv*d floats each,
 * either may be NULL), in the cache's own layout.  Synchronous. */
int zwg_kv_read(zwg_kv *kv, uint64_t layer, uint64_t seq, float *k_host, float *v_host);

/*
 * Linear layers: the drop-in for ops.linear (src/ops.zig:283-306) with f16 weights, the encoder's
 * Q/K/V/O projections and MLP (src/encoder.zig:164-174), BERT's (src/bert.zig:223-232) and the
 * scene model's (src/scene.zig:369-378).  out[i][o] = sum_p x[i][p] * w[o][p] (+ bias[o]), with
 * x f32 [m][k], w [n][k] of type w_type, bias f32 [n] or NULL, out f32 [m][n].
 * Computed on f16 MFMA with each x split into two f16 terms (f32-level accuracy; |x| must be
 * within f16's range, 65504, or its output row turns inf).  k a multiple of 8; pointers 16-byte
 * aligned.  A call with too few output tiles to fill the GPU and a long k splits k and keeps the
 * partial sums in the context's workspace (as many splits as fit); the splits are added in a
 * fixed order, so results do not vary from call to call.
 */
#define ZWG_W_F16 1u /* IEEE binary16 weights, as src/encoder.zig loads them */

/* Host pointers, synchronous: the drop-in for ops.linear.  Stages x, w, bias and out through
 * the context. */
int zwg_linear(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
               const float *bias, uint64_t n, float *out);
/* Device pointers, asynchronous on the context's stream. */
int zwg_linear_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
                   const float *bias, uint64_t n, float *out);

/*
 * Linear layers over int8 block weights: the drop-in for ops.linear with a gemm.Q8
 * (src/ops.zig:283-306, src/gemm.zig:188-351 -- ntBlockQ :330-351, micro4x4Q :289-327,
 * dotQ :274-286), the Whisper decoder's projections, MLP and logits (src/decoder.zig:181-205)
 * and cross K/V (:151-159), and Qwen2's q/k/v/o, gate/up/down and output (src/llm.zig:179-216).
 * q: int8 [n][k], scales: f32 [n][k / 32] (the Q8 struct's two arrays, as Q8.quantize and
 * Q8.fromQ8_0 build them, src/gemm.zig:209-248):
 *     out[i][o] = sum_b scales[o][b] * sum_{p in 32-block b} x[i][p] * q[o][p]  (+ bias[o])
 * k a multiple of 32 (the Q8 assertion, src/gemm.zig:210); x, q and out 16-byte aligned, scales
 * 4-byte aligned; |x| within f16's range (x is split into two f16 terms for the f16 MFMA, int8
 * weights are exact in f16).  m <= 64 (token steps) streams the weights once from HBM.
 */
#define ZWG_W_Q8 2u /* int8 block weights + f32 block scales (zwg_linear_q8*) */

/* Host pointers, synchronous. */
int zwg_linear_q8(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const int8_t *q, const float *scales,
                  const float *bias, uint64_t n, float *out);
/* Device pointers, asynchronous on the context's stream. */
int zwg_linear_q8_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const int8_t *q, const float *scales,
                      const float *bias, uint64_t n, float *out);

/*
 * Device-resident int8 block weights.  The reference builds each gemm.Q8 once at load
 * (Q8.quantize / Q8.fromQ8_0, src/gemm.zig:209-248; src/decoder.zig:203-215 getQ, src/llm.zig
 * loaders) and every forward then calls ops.linear with it.  zwg_q8w_create is that load step for
 * the GPU: it copies the Q8's two arrays into HBM once, repacked so that the token-step kernel
 * reads every weight byte in contiguous 1 KB wave-loads (tiles of 32 rows x 32 k in lane order,
 * scales grouped per 32 rows; zero padding to 32 rows and 256 k).  zwg_linear_q8w_dev computes
 * exactly what zwg_linear_q8_dev computes with the unpacked arrays.  zwg_close of the context
 * frees the packed copy of weights not destroyed yet; such weights then only accept
 * zwg_q8w_destroy (calls that use them fail).
 */
typedef struct zwg_q8w zwg_q8w;
#define ZWG_Q8W_FROM_HOST 1u /* q and scales are host memory (else device memory) */

/* q int8 [n][k], scales f32 [n][k / 32]; k a multiple of 32.  Returns when the packed copy is
 * done for host sources; device sources are packed asynchronously on ctx's stream. */
int zwg_q8w_create(zwg_ctx *ctx, const int8_t *q, const float *scales, uint64_t n, uint64_t k, uint32_t flags,
                   zwg_q8w **out);
void zwg_q8w_destroy(zwg_q8w *w);
int zwg_q8w_shape(const zwg_q8w *w, uint64_t *n, uint64_t *k);
/* out[m][n] = x[m][k] . W^T (+ bias): device pointers, asynchronous on ctx's stream. */
int zwg_linear_q8w_dev(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, const float *bias, float *out);

/*
 * Linear-layer epilogues: the value v = x . W^T + b of out[i][o] is stored as v (NONE), as gelu(v)
 * (GELU: ops.linear then ops.gelu, src/encoder.zig:172-173, src/decoder.zig:198-199), or added to
 * what out holds (ADD: ops.linear then ops.add, the residual of src/encoder.zig:169, :174).
 */
#define ZWG_EPI_NONE 0u
#define ZWG_EPI_GELU 1u
#define ZWG_EPI_ADD 2u

/* f16 weights with an epilogue and an output row stride (out_stride >= n; 0 = n),
 * device pointers, asynchronous. */
int zwg_linear_epi_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
                       const float *bias, uint64_t n, float *out, uint64_t out_stride, uint32_t epilogue);
/* Resident int8 weights with an epilogue, device pointers, asynchronous. */
int zwg_linear_q8w_epi_dev(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, const float *bias, float *out,
                           uint32_t epilogue);

/*
 * Several linear layers over the same x at once: out[j] = x . w[j]^T (+ bias[j]) for n_w (1..4)
 * resident weight sets that share k -- a decode step's q/k/v projections, or its MLP gate and up.
 * bias may be NULL, or hold NULL entries.  For m <= 64 the sets share one x split, one
 * weight-streaming launch and one split sum (three launches in all instead of three per set);
 * larger m runs the sets one after another.  Results equal the single calls' to f32 rounding (the
 * k split may differ).  No counterpart in the reference, which calls ops.linear
 * (src/ops.zig:283-306) once per projection (src/llm.zig:179-207, src/decoder.zig:181-201).
 */
int zwg_linear_q8w_group_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint32_t n_w, const zwg_q8w *const *w,
                             const float *const *bias, float *const *out);

/*
 * A decode step's q/k/v projections with the cache append in their final store: the projections
 * of zwg_linear_q8w_group_dev over w[0] (q: n_head * d rows), w[1] and w[2] (k, v: n_head_kv * d
 * rows of kv), bias[0..2] (each NULL or 16-byte aligned; bias itself may be NULL), then what
 * zwg_kv_append_batch(kv, layer, seq0, m, pos_dev, k, v, q_out, n_head, n_head * d) does with them:
 * with the cache's rotary tables q and k rotated at their token's position; q written to q_out
 * [m][n_head * d]; token i's k and v written into sequence seq0 + i's cache at pos_dev[i] (k
 * transposed for ZWG_KV_KT); a position outside [0, n_ctx) writes no cache rows and leaves q
 * unrotated.  q_out and the caches equal those two calls' bit for bit whenever the group call
 * splits k (its m <= 64 calls of fewer than 128 workgroups, which include the Whisper and Qwen2
 * decode steps' q/k/v); this call always splits, so the rows never go through memory unsummed.
 * m <= 64 (one row per sequence), k above 256.  As the reference, whose decoder writes the k and v
 * projections straight into its cache rows (src/decoder.zig:181-183) and whose Qwen2 step rotates
 * and scatters them (src/llm.zig:179-190): one launch fewer per layer than projections + append.
 * Device pointers, asynchronous.
 */
int zwg_linear_q8w_qkv_kv_dev(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *const *w,
                              const float *const *bias, float *q_out, zwg_kv *kv, uint64_t layer, uint64_t seq0,
                              const int32_t *pos_dev);

/*
 * Row-wise and elementwise ops around the projections, device pointers, asynchronous:
 * ops.layerNormEps (src/ops.zig:388-395; ops.layerNorm is eps = 1e-5, BERT uses 1e-12):
 * out[i] = (x[i] - mean) / sqrt(var + eps) * w + b per row of x [m][n]; ops.gelu (src/ops.zig:
 * 310-340), ggml's tanh form, in place; ops.add: x += y.  n and count multiples of 4, buffers
 * 16-byte aligned.
 */
int zwg_layer_norm_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, const float *b, float eps,
                       float *out);
int zwg_gelu_dev(zwg_ctx *ctx, float *x, uint64_t count);
int zwg_add_dev(zwg_ctx *ctx, float *x, const float *y, uint64_t count);
/* Qwen2's norm and MLP gate (src/llm.zig:178, :204-205): ops.rmsNorm (src/ops.zig:409-427),
 * out[i] = x[i] / sqrt(sum(x[i]^2) / n + eps) * w per row of x [m][n]; ops.siluMul
 * (src/ops.zig:429-439), gate = gate / (1 + e^-gate) * up in place (e^x the device's expf, the
 * reference's expVec polynomial agreeing to a few f32 ulps).  n and count multiples of 4, buffers
 * 16-byte aligned, device pointers, asynchronous. */
int zwg_rms_norm_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t n, const float *w, float eps, float *out);
int zwg_silu_mul_dev(zwg_ctx *ctx, float *gate, const float *up, uint64_t count);

/*
 * One Whisper encoder layer (the loop body of Encoder.encode, src/encoder.zig:164-175) over
 * n_windows windows at once: x [n_windows][n_ctx][n_state] is updated in place, as the
 * reference updates e.x.  Weights are the layer's tensors as src/encoder.zig loads them: f16
 * matrices [out][in], f32 norms and biases (k has no bias).  scratch: device memory of
 * zwg_encoder_layer_scratch(n_windows * n_ctx, n_state) floats (the reference's x_ln, q, k, v,
 * attn and hidden buffers, src/encoder.zig:98-106).  Device pointers, asynchronous.
 */
typedef struct zwg_enc_layer {
    const float *attn_ln_w, *attn_ln_b; /* [n_state] */
    const void *q_w;                    /* f16 [n_state][n_state] */
    const float *q_b;
    const void *k_w; /* no bias */
    const void *v_w;
    const float *v_b;
    const void *o_w;
    const float *o_b;
    const float *mlp_ln_w, *mlp_ln_b;
    const void *mlp0_w; /* f16 [4 n_state][n_state] */
    const float *mlp0_b;
    const void *mlp1_w; /* f16 [n_state][4 n_state] */
    const float *mlp1_b;
} zwg_enc_layer;

uint64_t zwg_encoder_layer_scratch(uint64_t n_rows, uint64_t n_state);
int zwg_encoder_layer_dev(zwg_ctx *ctx, float *x, uint64_t n_windows, uint64_t n_ctx, uint64_t n_state,
                          uint64_t n_head, const zwg_enc_layer *w, float *scratch);

/*
 * The Whisper text decoder on the device: Decoder.setAudio (src/decoder.zig:151-159) and
 * Decoder.forward (src/decoder.zig:165-205) for a batch of windows decoded in lockstep, one new
 * token per window per step.  The weights are the tensors src/decoder.zig:96-131 loads: int8
 * block matrices as resident zwg_q8w [out][in], f32 device vectors for norms and biases (a NULL
 * bias adds nothing).  The windows are the sequences of two zwg_kv caches, both ZWG_KV_ROW with
 * n_head_kv = n_head, d = n_state / n_head (32, 64 or 128) and no rotary positions: self_kv with
 * n_ctx = n_text_ctx (the reference's cache_k / cache_v, src/decoder.zig:39-40), cross_kv with
 * n_ctx = n_audio_ctx (cross_k / cross_v, :41-42); both hold at least n_layer layers.
 * n_state: a multiple of 4, above 256 and at most 2048.
 */
typedef struct zwg_dec_layer {
    const float *attn_ln_w, *attn_ln_b; /* [n_state] */
    const zwg_q8w *q_w;                 /* [n_state][n_state] */
    const float *q_b;
    const zwg_q8w *k_w; /* no bias */
    const zwg_q8w *v_w;
    const float *v_b;
    const zwg_q8w *o_w;
    const float *o_b;
    const float *cross_ln_w, *cross_ln_b;
    const zwg_q8w *cq_w;
    const float *cq_b;
    const zwg_q8w *ck_w; /* no bias; used by zwg_decoder_set_audio_dev */
    const zwg_q8w *cv_w;
    const float *cv_b;
    const zwg_q8w *co_w;
    const float *co_b;
    const float *mlp_ln_w, *mlp_ln_b;
    const zwg_q8w *mlp0_w; /* [4 n_state][n_state] */
    const float *mlp0_b;
    const zwg_q8w *mlp1_w; /* [n_state][4 n_state] */
    const float *mlp1_b;
} zwg_dec_layer;

typedef struct zwg_decoder {
    uint64_t n_vocab, n_state, n_head, n_layer;
    const zwg_q8w *te;           /* token embedding [n_vocab][n_state], also the logits' weights */
    const float *pe;             /* positional embedding [n_text_ctx][n_state] */
    const float *ln_w, *ln_b;    /* the final layer norm */
    const zwg_dec_layer *layers; /* host array of n_layer */
    zwg_kv *self_kv;
    zwg_kv *cross_kv;
} zwg_decoder;

/* setAudio for windows seq0 .. seq0 + n_windows - 1: enc [n_windows][n_audio_ctx][n_state] (the
 * encoder's output, device) projected by every layer's ck_w and cv_w (+ cv_b) straight into the
 * windows' cross caches.  Asynchronous. */
int zwg_decoder_set_audio_dev(zwg_ctx *ctx, const zwg_decoder *dec, const float *enc, uint64_t n_windows,
                              uint64_t seq0);

/* Floats of scratch a step over m windows needs (the reference's x, x_ln, q, attn and hidden
 * buffers, src/decoder.zig:57-63, the cross-attention query's k-split partial sums and the
 * self-attention key counts). */
uint64_t zwg_decoder_scratch(uint64_t m, uint64_t n_state);

/* forward for windows seq0 .. seq0 + m - 1 (m <= 64), window i taking token tokens[i] at
 * position pos[i] (its n_past; tokens, pos: device int32 [m]): embeddings, every layer (its k and
 * v rows written into the self cache at pos[i], self-attention over the window's pos[i] + 1
 * cached keys, cross-attention over all n_audio_ctx keys), the final layer norm and the logits
 * [m][n_vocab] = ln(x) . te^T.  A position outside [0, n_text_ctx) writes no cache rows and its
 * window's logits are meaningless; a token outside [0, n_vocab) embeds as a zero row.  The work
 * the reference does, fused where it saves launches (layer norms into the residual projections'
 * split sums, the cache writes into the q/k/v projections', the cross-attention query's split sum
 * into the attention's query load), with results equal bit for bit to
 * the same step composed of zwg_layer_norm_dev, zwg_linear_q8w_qkv_kv_dev,
 * zwg_attention_batch_dev and zwg_linear_q8w_epi_dev calls.  Asynchronous. */
int zwg_decoder_step_dev(zwg_ctx *ctx, const zwg_decoder *dec, const int32_t *tokens, const int32_t *pos, uint64_t m,
                         uint64_t seq0, float *logits, float *scratch);

/*
 * Qwen2's decode step on the device: Model.forward (src/llm.zig:169-216) with one new token in
 * each of m sequences decoded in lockstep.  Weights as src/llm.zig:104-126 loads them: int8
 * block matrices as resident zwg_q8w [out][in], f32 device vectors for norms and biases (a NULL
 * bias adds nothing); `output` may be `embd` (tied).  The sequences are those of one zwg_kv,
 * ZWG_KV_KT with n_head_kv, d = n_embd / n_head (32, 64 or 128) and the model's rotary base
 * (qwen2.rope.freq_base), holding at least n_layer layers: the reference's cache_kt and cache_v
 * (src/llm.zig:27-29).  n_embd a multiple of 4, above 256 and at most 4096; n_ff a multiple of 4.
 */
typedef struct zwg_llm_layer {
    const float *attn_norm; /* [n_embd] */
    const zwg_q8w *wq;      /* [n_embd][n_embd] */
    const float *bq;
    const zwg_q8w *wk; /* [n_head_kv * d][n_embd] */
    const float *bk;
    const zwg_q8w *wv;
    const float *bv;
    const zwg_q8w *wo; /* [n_embd][n_embd], no bias */
    const float *ffn_norm;
    const zwg_q8w *w_gate; /* [n_ff][n_embd] */
    const zwg_q8w *w_up;
    const zwg_q8w *w_down; /* [n_embd][n_ff] */
} zwg_llm_layer;

typedef struct zwg_llm {
    uint64_t n_vocab, n_embd, n_head, n_head_kv, n_ff, n_layer;
    float eps;         /* qwen2.attention.layer_norm_rms_epsilon (src/llm.zig:100) */
    uint32_t reserved; /* must be 0 */
    const zwg_q8w *embd;   /* [n_vocab][n_embd] */
    const zwg_q8w *output; /* [n_vocab][n_embd] */
    const float *output_norm;
    const zwg_llm_layer *layers; /* host array of n_layer */
    zwg_kv *kv;
} zwg_llm;

/* Floats of scratch a step over m sequences needs (the reference's x, h, q, attn, gate and up
 * buffers, src/llm.zig:139-146, the attention's key counts and the ffn-normed rows split into f16
 * halves for the gate/up projections). */
uint64_t zwg_llm_scratch(uint64_t m, uint64_t n_embd, uint64_t n_ff);

/* forward for sequences seq0 .. seq0 + m - 1 (m <= 64), sequence i taking token tokens[i] at
 * position pos[i] (its n_past; device int32 [m]): embedding, every layer (q and k rotated at
 * pos[i], k scattered into the transposed cache and v into its rows, attention over the pos[i] +
 * 1 cached keys, the SiLU-gated MLP), the output norm and the logits [m][n_vocab].  A position
 * outside [0, n_ctx) writes no cache rows and its sequence's logits are meaningless; a token
 * outside [0, n_vocab) embeds as a zero row.  The RMS norms are fused into the residual
 * projections' split sums and the cache writes into the q/k/v projections', with results equal
 * bit for bit to the same step composed of zwg_rms_norm_dev, zwg_linear_q8w_qkv_kv_dev,
 * zwg_attention_batch_dev, zwg_linear_q8w_epi_dev, zwg_linear_q8w_group_dev and
 * zwg_silu_mul_dev calls.  Asynchronous. */
int zwg_llm_step_dev(zwg_ctx *ctx, const zwg_llm *lm, const int32_t *tokens, const int32_t *pos, uint64_t m,
                     uint64_t seq0, float *logits, float *scratch);

/* Floats of scratch a zwg_llm_forward_dev call over n tokens needs. */
uint64_t zwg_llm_forward_scratch(uint64_t n, uint64_t n_embd, uint64_t n_ff);

/*
 * Qwen2's Model.forward (src/llm.zig:169-216) over n tokens of one sequence, the reference's
 * prompt batch (Model.prompt, src/llm.zig:258-266, feeds a prompt in such batches): tokens[n]
 * (device int32) at positions pos0 .. pos0 + n - 1 of sequence seq of lm->kv (pos0 + n <=
 * n_ctx), written into the cache at those positions; logits[n_vocab] (device) are the last
 * token's.  Each step is the library call of the reference's op (rmsNorm, the grouped q/k/v
 * projections, zwg_kv_append with q, zwg_attention_dev causal over the pos0 + n cached keys, the
 * int8 linears with the residual add in their store, siluMul), so a token's results match the
 * one-token step's within f32 rounding (other kernels, other summation orders).  scratch:
 * zwg_llm_forward_scratch(n, ...) floats, 16-byte aligned; the attention's key-split partials
 * use the context's workspace.  Asynchronous.
 */
int zwg_llm_forward_dev(zwg_ctx *ctx, const zwg_llm *lm, const int32_t *tokens, uint64_t n, uint64_t seq,
                        uint64_t pos0, float *logits, float *scratch);

int zwg_version(void); /* ZWG_VERSION */

#ifdef __cplusplus
}
#endif
#endif /* ZW_GPU_H */
