// Linear layers around attention on gfx950 MFMA (include/zw_gpu.h, zwg_linear*).
//
// Replaces ops.linear (src/ops.zig:283-306): out[i][o] = sum_p x[i][p] * w[o][p] (+ b[o]), x f32
// [m][k], w logically [n][k] as the reference keeps it, over the register-blocked broadcast-FMA
// kernels of src/gemm.zig.
//   * f16 weights (ntBlock / micro4x4 / dot1, src/gemm.zig:117-137): the encoder's Q/K/V/O
//     projections and MLP (src/encoder.zig:164-174), BERT (src/bert.zig:223-232), the scene
//     model (src/scene.zig:369-378).
//   * int8 block weights (gemm.Q8, ntBlockQ / micro4x4Q / dotQ, src/gemm.zig:188-351): the
//     Whisper decoder's projections, MLP and logits (src/decoder.zig:181-205) and cross K/V
//     (:151-159), Qwen2's q/k/v/o, gate/up/down and output (src/llm.zig:179-216).
// The kernels, their precision and tiling are described in linear_kernel.hpp and
// linear_q8_kernel.hpp.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <string>

#include "linear_kernel.hpp"
#include "linear_q8_kernel.hpp"
#include "elementwise.hpp"
#include "zw_ctx.hpp"
#include "zw_gpu.h"

using namespace zwg_host;
using zwg_lin::LinearArgs;

namespace {

int64_t tiles(uint64_t m, uint64_t n, int bm, int bn) { return (int64_t)((m + bm - 1) / bm) * (int64_t)((n + bn - 1) / bn); }

// Tile choice (swept on the device over the encoder, decoder and Qwen2 projection shapes): the
// 128 x 256 tile when it gives two workgroups per CU (256 CUs), else 64 x 256 when that fills
// the CUs once, else 64 x 64 for the small single-window shapes, which are latency bound.  Int8
// weights take 128 x 128 in place of 128 x 256: the block sums need 16 more VGPRs per tile row,
// which would leave the larger tile one wave per SIMD.  The x 256 tiles run 8 waves (2 x 4):
// half the accumulators and staging registers per wave (76 and 124 VGPRs against 141 and 235),
// so LDS rather than registers sets the occupancy -- twice the waves per SIMD, which hides more
// of the per-stage load latency (measured 6-7% on the base.en projections and layer).
// Threads per workgroup of the short element-wise kernels around the int8 and split paths (the
// x split, the split sums): 64 when the call has fewer than 1024 workgroups' worth at 256, so a
// small call's one round of loads comes from every CU rather than a few (as the attention merge)
inline int small_block(int64_t threads) { return threads < 1024ll * 256 ? 64 : 256; }
inline unsigned blocks_for(int64_t threads, int bs) { return (unsigned)((threads + bs - 1) / bs); }

// The split sum of n_split partial products part[s][m][n] into out (row stride ldo)
hipError_t launch_split_sum(const float *part, const float *bias, float *out, int64_t mn, int32_t n, int n_split,
                            uint32_t epi, int64_t ldo, hipStream_t stream) {
    if (n % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15) == 0) {
        const int64_t threads = mn / 4;
        const int bs = small_block(threads);
        zwg_lin::linear_split_sum_kernel<4><<<blocks_for(threads, bs), bs, 0, stream>>>(
            part, bias, out, mn, n, n_split, epi, ldo);
    } else {
        const int bs = small_block(mn);
        zwg_lin::linear_split_sum_kernel<1><<<blocks_for(mn, bs), bs, 0, stream>>>(
            part, bias, out, mn, n, n_split, epi, ldo);
    }
    return hipGetLastError();
}

struct TileChoice {
    int bm, bn;
};
template <int WMODE>
TileChoice choose_tile(uint64_t m, uint64_t n) {
    if constexpr (WMODE != zwg_lin::kWF16) {
        if (tiles(m, n, 128, 128) >= 512) return {128, 128};
    } else {
        if (tiles(m, n, 128, 256) >= 512) return {128, 256};
    }
    if (tiles(m, n, 64, 256) >= 256) return {64, 256};
    return {64, 64};
}

template <int WMODE>
hipError_t launch_tiled(const LinearArgs &a, TileChoice tc, int n_split, hipStream_t stream) {
    if constexpr (WMODE != zwg_lin::kWF16) {
        if (tc.bm == 128) return zwg_lin::launch_linear_tile<128, 128, WMODE>(a, n_split, stream);
    } else {
        if (tc.bm == 128) return zwg_lin::launch_linear_tile<128, 256, WMODE, 4>(a, n_split, stream);
    }
    if (tc.bn == 256) return zwg_lin::launch_linear_tile<64, 256, WMODE, 4>(a, n_split, stream);
    if (n_split > 1) return zwg_lin::launch_linear_tile<64, 64, WMODE, 2, true>(a, n_split, stream);
    return zwg_lin::launch_linear_tile<64, 64, WMODE>(a, n_split, stream);
}

// A call with fewer tiles than two per CU and a long k (prefill batches of a few hundred rows
// through a wide MLP, single windows) splits k over more workgroups, about 512 in all, as long as
// the partial sums fit the workspace; a second kernel adds the splits in a fixed order, so results
// stay deterministic.  Each split keeps at least 16 stages of 32 (8 below 64 tiles, where the
// fill gained outweighs everything): shorter splits measured slower than none, the partials'
// round trip and second launch costing more than the extra workgroups hide.  Only 64 x 64 tiles
// split (a wider tile is chosen only when there would be 1024 or more 64 x 64 tiles, twice what a
// split aims for), and the split kernel is an instantiation of its own, so the unsplit one is
// compiled exactly as without it.
template <int WMODE>
int run_tiled(zwg_ctx *ctx, LinearArgs a) {
    const TileChoice tc = choose_tile<WMODE>((uint64_t)a.m, (uint64_t)a.n);
    const int64_t n_tiles = tiles((uint64_t)a.m, (uint64_t)a.n, tc.bm, tc.bn);
    const int stages = (a.k + zwg_lin::BK - 1) / zwg_lin::BK;
    const uint64_t mn = (uint64_t)a.m * (uint64_t)a.n;
    int n_split = 1;
    if (tc.bn == 64 && n_tiles < 512 && stages >= 16) {
        n_split = (int)std::min<int64_t>((512 + n_tiles - 1) / n_tiles, stages / (n_tiles < 64 ? 8 : 16));
        while (n_split > 1 && (uint64_t)n_split * mn * 4 > ctx->workspace_bytes) --n_split;
    }
    const int split_stages = (stages + n_split - 1) / n_split;
    a.k_split = split_stages * zwg_lin::BK;
    n_split = (stages + split_stages - 1) / split_stages; // no empty splits
    a.part = n_split > 1 ? reinterpret_cast<float *>(ctx->workspace) : nullptr;
    hipError_t e = launch_tiled<WMODE>(a, tc, n_split, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "linear kernel launch", e);
    if (n_split > 1) {
        e = launch_split_sum(a.part, a.bias, a.out, (int64_t)mn, a.n, n_split, a.epi, a.ldo, ctx->stream);
        if (e != hipSuccess) return fail_hip(ctx, "linear split-sum kernel launch", e);
    }
    return ZWG_OK;
}

std::string check_linear(uint64_t m, uint64_t k, uint32_t w_type, uint64_t n) {
    if (w_type != ZWG_W_F16 && w_type != ZWG_W_Q8) return "w_type must be ZWG_W_F16 or ZWG_W_Q8";
    if (k == 0 || k % 8) return "k must be a positive multiple of 8";
    if (w_type == ZWG_W_Q8 && k % 32) return "k must be a multiple of 32 for int8 block weights";
    if (m > 0x7fffffffull || n > 0x7fffffffull || k > 0x7fffffffull) return "m, n and k must be below 2^31";
    if ((n + 63) / 64 > 65535) return "n too large (above 65535 x 64)";
    if (k > (1ull << 20)) return "k above 2^20";  // keeps a workgroup's buffer range below 2^31 bytes
    return "";
}

// Q8 with m <= 64: x split into hi/lo halves by linear_q8_xprep_kernel into the workspace, then
// the weight-streaming kernel.  Four waves of S slabs of 32 weight rows per workgroup (S = 2 when
// that alone makes >= 256 workgroups, else 1); a call of fewer than 512 workgroups splits k over
// more, at chunk granularity, up to about ZWG_Q8P_SPLIT_TARGET of them, as long as the partial
// sums fit the workspace.  (Raw-layout weights; the resident packed ones go through run_q8p_group.)
//
// Workgroups a split call is split up to (within its k chunks).  Only the Qwen2.5-1.5B down
// projection (k = 8960: 18-way at 256, 35-way at 512) reaches it; its projections alone measured
// 2163 / 2048 / 1960 / 1964 / 1963 us at 128 / 192 / 256 / 512 / 1024, and its whole token step,
// whose down projection's sums add into x and normalise it in one row kernel, 4.117 / 4.073 /
// 4.074 ms at 512 / 384 / 256 (paired runs): that kernel reads half the partials at 256
#ifndef ZWG_Q8P_SPLIT_TARGET
#define ZWG_Q8P_SPLIT_TARGET 256
#endif
template <int MT>
int run_q8_stream_mt(zwg_ctx *ctx, const zwg_lin::Q8Args &base) {
    zwg_lin::Q8Args a = base;
    const uint64_t m = (uint64_t)a.m, n = (uint64_t)a.n;
    const int S = (n + 255) / 256 >= 256 ? 2 : 1;
    const int64_t gx = (int64_t)((n + 128 * S - 1) / (128 * S));
    const int n_chunks = (a.k + zwg_lin::kQ8Chunk - 1) / zwg_lin::kQ8Chunk;
    const uint64_t xcvt_bytes = (uint64_t)n_chunks * zwg_lin::q8_chunk_halves<MT>() * 2;
    const uint64_t part_off = (xcvt_bytes + 255) / 256 * 256;
    if (part_off > ctx->workspace_bytes) return fail(ctx, "workspace too small for this linear call");
    int n_split = 1;
    // split up to the packed calls' target, so both layouts split a call into the same pieces
    if (gx < 512) n_split = (int)std::min<int64_t>(n_chunks, (ZWG_Q8P_SPLIT_TARGET + gx - 1) / gx);
    while (n_split > 1 && part_off + (uint64_t)n_split * m * n * 4 > ctx->workspace_bytes) --n_split;
    a.chunks_per_split = (n_chunks + n_split - 1) / n_split;
    n_split = (n_chunks + a.chunks_per_split - 1) / a.chunks_per_split; // no empty splits
    a.n_split = n_split;
    _Float16 *xcvt = reinterpret_cast<_Float16 *>(ctx->workspace);
    a.part = n_split > 1 ? reinterpret_cast<float *>(reinterpret_cast<char *>(ctx->workspace) + part_off) : nullptr;

    const int64_t prep_threads = (int64_t)n_chunks * MT * 32 * (zwg_lin::kQ8Chunk / 4);
    const int prep_bs = small_block(prep_threads);
    zwg_lin::linear_q8_xprep_kernel<MT><<<blocks_for(prep_threads, prep_bs), prep_bs, 0, ctx->stream>>>(
        a.x, xcvt, a.m, a.k, n_chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail_hip(ctx, "linear (int8) x preparation launch", e);
    dim3 grid((unsigned)gx, (unsigned)n_split);
    if (S == 2) zwg_lin::linear_q8_stream_kernel<MT, 2><<<grid, zwg_lin::kQ8Threads, 0, ctx->stream>>>(a, xcvt);
    else zwg_lin::linear_q8_stream_kernel<MT, 1><<<grid, zwg_lin::kQ8Threads, 0, ctx->stream>>>(a, xcvt);
    e = hipGetLastError();
    if (e != hipSuccess) return fail_hip(ctx, "linear (int8 stream) kernel launch", e);
    if (n_split > 1) {
        const int64_t mn = (int64_t)(m * n);
        e = launch_split_sum(a.part, a.bias, a.out, mn, (int32_t)n, n_split, a.epi, (int64_t)n, ctx->stream);
        if (e != hipSuccess) return fail_hip(ctx, "linear split-sum kernel launch", e);
    }
    return ZWG_OK;
}

// Resident packed weights with m <= 64, one or more weight sets over the same x (g.count sets;
// q/scales/n_slabs/n/bias/out filled by the caller): one stream launch over every set's
// workgroups (four slabs of 32 rows each), preceded by one x split for 64-row calls (32-row calls
// split x inside the stream kernel), and when k is split, one split sum over every set's outputs.
// The k split is chosen from the group's total workgroup count, as for a single call: a call of
// fewer than ZWG_Q8P_SPLIT_BELOW workgroups is split until it has about 512.
#ifndef ZWG_Q8P_WAVES
#define ZWG_Q8P_WAVES 4
#endif
#ifndef ZWG_Q8P_WAVES_32
#define ZWG_Q8P_WAVES_32 2
#endif
// waves (one 32-row slab each) sharing each x stage of the packed stream kernel: four for 64-row
// calls (8 measured 5-9% slower on the logits and decode-step workloads: half the workgroups,
// longer tails; 2 measured 4% slower on the Qwen2.5-1.5B step and 26% on its logits), two for
// 32-row calls, whose x stage is half as large (Whisper small.en step 675 -> 651 us against 4)
template <int MT>
constexpr int q8p_waves() { return MT == 1 ? ZWG_Q8P_WAVES_32 : ZWG_Q8P_WAVES; }
// k is split only for calls below this many workgroups.  A call at or above it streams unsplit:
// its partial sums would be as large as half its weights (the Qwen2.5-1.5B gate/up, 140
// workgroups: split 3 ways, 13.8 MB of partials for 27.5 MB of weights).  Measured on one box,
// splitting below 512 / 160 / 100 / 64 workgroups: Qwen2.5-1.5B decode step 2297 / 2297 / 2126 /
// 2118 us, small.en decoder step 690 / 675 / 675 / 675 us.
#ifndef ZWG_Q8P_XS_SPLIT
#define ZWG_Q8P_XS_SPLIT 1
#endif
#ifndef ZWG_Q8P_SPLIT_BELOW
#define ZWG_Q8P_SPLIT_BELOW 128
#endif
// unsplit calls of fewer workgroups than this run two stage groups per workgroup (each over half
// of k, summed through LDS at the end)
#ifndef ZWG_Q8P_KS_BELOW
#define ZWG_Q8P_KS_BELOW 256
#endif
// calls of up to this many rows stream the resident weights (64-row blocks of one launch); more
// rows take the tiled GEMM
#ifndef ZWG_Q8P_STREAM_ROWS
#define ZWG_Q8P_STREAM_ROWS 256
#endif


// Row kernels of n <= 2048 floats (a wave per row, n / 256 float4 per lane, rounded up), one
// wave per workgroup: a decode step's few rows then read their partials through as many CUs as
// there are rows (four rows per workgroup put a 32-row step's 1.3 MB of partial loads through 8
// CUs' load paths)
constexpr int kMaxRowN = 4096; // the row kernels' widest row: 16 float4 per lane
template <template <int, int> class K, int NORM, typename... Args>
hipError_t launch_rows(int32_t n, int32_t m, hipStream_t stream, Args... args) {
    const int R = (n / 4 + 63) / 64;
    const dim3 grid((unsigned)m), block(64);
    switch (R) {
    case 1: K<1, NORM>::launch(grid, block, stream, args...); break;
    case 2: K<2, NORM>::launch(grid, block, stream, args...); break;
    case 3: K<3, NORM>::launch(grid, block, stream, args...); break;
    case 4: K<4, NORM>::launch(grid, block, stream, args...); break;
    case 5: K<5, NORM>::launch(grid, block, stream, args...); break;
    case 6: K<6, NORM>::launch(grid, block, stream, args...); break;
    case 7: K<7, NORM>::launch(grid, block, stream, args...); break;
    case 8: K<8, NORM>::launch(grid, block, stream, args...); break;
    case 10: K<10, NORM>::launch(grid, block, stream, args...); break;
    case 12: K<12, NORM>::launch(grid, block, stream, args...); break;
    case 14: K<14, NORM>::launch(grid, block, stream, args...); break;
    case 9: case 11: case 13: case 15: case 16: K<16, NORM>::launch(grid, block, stream, args...); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
template <int R, int NORM>
struct AddLnRows {
    static void launch(dim3 g, dim3 b, hipStream_t st, const float *part, const float *bias, zwg_lin::Q8ResLn r,
                       int32_t m, int32_t n, int32_t n_split) {
        zwg_lin::linear_split_sum_add_ln_kernel<R, NORM><<<g, b, 0, st>>>(part, bias, r, m, n, n_split);
    }
};
template <int R, int NORM>
struct AddLnWideRows { // R waves per row: the block size is the kernel's own
    static void launch(dim3 g, dim3, hipStream_t st, const float *part, const float *bias, zwg_lin::Q8ResLn r,
                       int32_t m, int32_t n, int32_t n_split) {
        zwg_lin::linear_split_sum_add_ln_wide_kernel<R, NORM><<<g, dim3(64 * R), 0, st>>>(part, bias, r, m, n, n_split);
    }
};
// the split sum + residual + norm kernel: one thread per float4 column (1) or one wave per row (0).
// Paired runs on one box, per step: Whisper small.en decoder (32 windows) 1563 -> 1537 us, Qwen2.5-1.5B
// decode (64 sequences; its down projection's sums take 35 splits) 4394 -> 4198 us.
#ifndef ZWG_ADDLN_WIDE
#define ZWG_ADDLN_WIDE 1
#endif
template <int R, int NORM>
using AddLnChosen = std::conditional_t<ZWG_ADDLN_WIDE != 0, AddLnWideRows<R, NORM>, AddLnRows<R, NORM>>;
template <int R, int NORM>
struct EmbedLnRows {
    static void launch(dim3 g, dim3 b, hipStream_t st, zwg_lin::Q8Packed te, int32_t n_vocab, const int32_t *tok,
                       const float *pe, const int32_t *pos, int32_t pe_rows, int32_t m, int32_t n, float *x,
                       zwg_lin::Q8ResLn r) {
        zwg_lin::q8p_embed_ln_kernel<R, NORM><<<g, b, 0, st>>>(te, n_vocab, tok, pe, pos, pe_rows, m, n, x, r);
    }
};

// kvs (a q/k/v group, sets 0, 1, 2): the split sum stores into q_out and the KV cache
// (linear_split_sum_qkv_kernel), so the call is always split, in two at least.  resln (one set,
// n <= 2048): the split sum adds into the residual stream and normalises the rows
// (linear_split_sum_add_ln_kernel), likewise always split.
// po (one set): the partials go to po->part (at most po->max_parts splits, at least two) and no
// split sum is launched; the split count is returned in po->n_split.
struct Q8PartsOut {
    float *part;
    int max_parts;
    int n_split;
};
// calls of several 64-row blocks (gridDim.z) take their own split rule: split below the same
// count, up to about 256 workgroups (the Qwen2.5-0.5B prompt's 256-row calls, per 2048-token
// prompt: 22.43 ms at 512, 22.19 at 256; splitting calls of up to 512 or 1024 workgroups: 23.9 ms)
#ifndef ZWG_Q8P_SPLIT_BELOW_Z
#define ZWG_Q8P_SPLIT_BELOW_Z ZWG_Q8P_SPLIT_BELOW
#endif
#ifndef ZWG_Q8P_SPLIT_TARGET_Z
#define ZWG_Q8P_SPLIT_TARGET_Z 256
#endif
bool q8p_split_k(int64_t gx, int n_chunks, int nz = 1) {
    return gx < (nz > 1 ? ZWG_Q8P_SPLIT_BELOW_Z : ZWG_Q8P_SPLIT_BELOW) && n_chunks > 1;
}
// 32-row calls split x inside the stream kernel; 64-row ones too when k is split (small calls,
// where the separate pass's launch costs more than the fused split), otherwise in a pass of their
// own first.
template <int MT>
bool q8p_splits_x_itself(int64_t gx, int n_chunks) {
    return MT == 1 || (ZWG_Q8P_XS_SPLIT && q8p_split_k(gx, n_chunks));
}
template <int MT>
int run_q8p_group(zwg_ctx *ctx, const zwg_lin::Q8Args &base, zwg_lin::Q8Group g,
                  const zwg_lin::Q8KvStore *kvs = nullptr, const zwg_lin::Q8ResLn *resln = nullptr,
                  Q8PartsOut *po = nullptr, const _Float16 *xcvt_in = nullptr) {
    constexpr int kQ8pWaves = q8p_waves<MT>();
    zwg_lin::Q8Args a = base;
    const uint64_t m = (uint64_t)a.m;
    const bool pair = g.swiglu != 0;
    if (pair && (g.count != 2 || g.n[0] != g.n[1] || kvs || resln || po))
        return fail(ctx, "a SwiGLU pair is two weight sets of the same shape, with no fused store");
    int64_t gx = 0;
    uint64_t n_tot = 0;
    for (int j = 0; j < zwg_lin::kQ8MaxGroup; ++j) {
        g.block_start[j] = (int32_t)gx;
        g.elem_start[j] = (int64_t)(m * n_tot);
        if (j < g.count) {
            gx += (g.n[j] + 32 * kQ8pWaves - 1) / (32 * kQ8pWaves);
            n_tot += (uint64_t)g.n[j];
        }
    }
    g.block_start[zwg_lin::kQ8MaxGroup] = (int32_t)gx;
    g.elem_start[zwg_lin::kQ8MaxGroup] = (int64_t)(m * n_tot);
    const int n_chunks = (a.k + zwg_lin::kQ8Chunk - 1) / zwg_lin::kQ8Chunk;
    g.n_chunks = n_chunks;
    // a SwiGLU pair's workgroups each take the same columns of both sets: the grid covers one
    // set's columns at half the rows per workgroup, while every choice below is the two sets'
    // unpaired one (so the sums are the same as the pair's two separate outputs')
    const int64_t gx_launch = pair ? ((int64_t)g.n[0] + 16 * kQ8pWaves - 1) / (16 * kQ8pWaves) : gx;
    // calls of more than 64 rows: nz blocks of 64 rows in one launch (gridDim.z), x split in the
    // kernel, and the k split chosen from all nz gx workgroups
    const int nz = (int)((m + 32 * MT - 1) / (32 * MT));
    if (nz > 1 && (MT != 2 || po || xcvt_in || (resln && resln->xcvt)))
        return fail(ctx, "the split rows and partials calls take at most 64 rows");
    const int64_t gxz = gx * nz;
    const bool split_k = q8p_split_k(gxz, n_chunks, nz);
    // xcvt_in (a 64-row call): x was split by the caller's previous launch.  The partial sums keep
    // the place (and so the split count) the call has without it.
    const bool xs_own = q8p_splits_x_itself<MT>(gxz, n_chunks) || nz > 1;
    const bool XS = xs_own && !(MT == 2 && xcvt_in);
    if (resln && resln->xcvt && (ZWG_ADDLN_WIDE == 0 || MT != 2))
        return fail(ctx, "split rows for the next call come from 33..64-row calls' one-thread-per-column sums");
    const uint64_t xcvt_bytes = xs_own ? 0 : (uint64_t)n_chunks * zwg_lin::q8_chunk_halves<MT>() * 2;
    const uint64_t part_off = (xcvt_bytes + 255) / 256 * 256;
    if (part_off > ctx->workspace_bytes) return fail(ctx, "workspace too small for this linear call");
    int n_split = 1;
    const int64_t target = nz > 1 ? ZWG_Q8P_SPLIT_TARGET_Z : ZWG_Q8P_SPLIT_TARGET;
    if (split_k) n_split = (int)std::min<int64_t>(n_chunks, (target + gxz - 1) / gxz);
    if (kvs || resln || po) {
        if (n_chunks < 2) return fail(ctx, "the fused split-sum calls need k above 256 (their sum is a k split)");
        n_split = std::max(n_split, 2);
    }
    if (po) n_split = std::min(n_split, po->max_parts);
    else while (n_split > 1 && part_off + (uint64_t)n_split * m * n_tot * 4 > ctx->workspace_bytes) --n_split;
    if ((kvs || resln || po) && n_split < 2) return fail(ctx, "too little room for this call's partial sums");
    a.chunks_per_split = (n_chunks + n_split - 1) / n_split;
    n_split = (n_chunks + a.chunks_per_split - 1) / a.chunks_per_split; // no empty splits
    a.n_split = n_split;
    char *ws = reinterpret_cast<char *>(ctx->workspace);
    uint64_t off = part_off;
    for (int j = 0; j < zwg_lin::kQ8MaxGroup; ++j) {
        g.part[j] = (j < g.count && n_split > 1) ? reinterpret_cast<float *>(ws + off) : nullptr;
        if (j < g.count) off += (uint64_t)n_split * m * (uint64_t)g.n[j] * 4;
    }
    if (po) {
        g.part[0] = po->part;
        po->n_split = n_split;
    }
    // xcvt_in: x already split in this layout by the previous call's row kernel
    const _Float16 *xcvt = XS ? nullptr : xcvt_in ? xcvt_in : reinterpret_cast<_Float16 *>(ctx->workspace);
    hipError_t e;
    if (!XS && !xcvt_in) {
        const int64_t prep_threads = (int64_t)n_chunks * MT * 32 * (zwg_lin::kQ8Chunk / 4);
        const int prep_bs = small_block(prep_threads);
        zwg_lin::linear_q8_xprep_kernel<MT><<<blocks_for(prep_threads, prep_bs), prep_bs, 0, ctx->stream>>>(
            a.x, reinterpret_cast<_Float16 *>(ctx->workspace), a.m, a.k, n_chunks);
        e = hipGetLastError();
        if (e != hipSuccess) return fail_hip(ctx, "linear (int8) x preparation launch", e);
    }
    dim3 grid((unsigned)gx_launch, (unsigned)n_split, (unsigned)nz);
    // unsplit calls of too few workgroups to fill the chip: two stage groups per workgroup
    const bool two_groups = n_split == 1 && gxz < ZWG_Q8P_KS_BELOW && n_chunks > 1;
    using namespace zwg_lin;
    constexpr int W = kQ8pWaves;
    if (pair) {
        if (two_groups) {
            if (XS) linear_q8p_stream_kernel<MT, 1, W, true, 2, true><<<grid, 128 * W, 0, ctx->stream>>>(a, g, xcvt);
            else linear_q8p_stream_kernel<MT, 1, W, false, 2, true><<<grid, 128 * W, 0, ctx->stream>>>(a, g, xcvt);
        } else {
            if (XS) linear_q8p_stream_kernel<MT, 1, W, true, 1, true><<<grid, 64 * W, 0, ctx->stream>>>(a, g, xcvt);
            else linear_q8p_stream_kernel<MT, 1, W, false, 1, true><<<grid, 64 * W, 0, ctx->stream>>>(a, g, xcvt);
        }
    } else if (two_groups) {
        if (XS) linear_q8p_stream_kernel<MT, 1, W, true, 2><<<grid, 128 * W, 0, ctx->stream>>>(a, g, xcvt);
        else linear_q8p_stream_kernel<MT, 1, W, false, 2><<<grid, 128 * W, 0, ctx->stream>>>(a, g, xcvt);
    } else {
        if (XS) linear_q8p_stream_kernel<MT, 1, W, true><<<grid, 64 * W, 0, ctx->stream>>>(a, g, xcvt);
        else linear_q8p_stream_kernel<MT, 1, W, false><<<grid, 64 * W, 0, ctx->stream>>>(a, g, xcvt);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return fail_hip(ctx, "linear (int8 stream) kernel launch", e);
    if (kvs) {
        const int64_t threads = (int64_t)m * (kvs->n_head + 2 * kvs->n_head_kv) * (kvs->d / 8);
        const int bs = small_block(threads);
        if (kvs->d == 64)
            zwg_lin::linear_split_sum_qkv_kernel<64><<<blocks_for(threads, bs), bs, 0, ctx->stream>>>(g, *kvs, a.m, n_split);
        else if (kvs->d == 128)
            zwg_lin::linear_split_sum_qkv_kernel<128><<<blocks_for(threads, bs), bs, 0, ctx->stream>>>(g, *kvs, a.m, n_split);
        else
            zwg_lin::linear_split_sum_qkv_kernel<32><<<blocks_for(threads, bs), bs, 0, ctx->stream>>>(g, *kvs, a.m, n_split);
        e = hipGetLastError();
        if (e != hipSuccess) return fail_hip(ctx, "q/k/v cache split-sum kernel launch", e);
    } else if (po) {
        // the caller adds the partials (attention's q load)
    } else if (resln) {
        e = resln->norm == zwg_ew::kNormRms
                ? launch_rows<AddLnChosen, zwg_ew::kNormRms>(g.n[0], a.m, ctx->stream, (const float *)g.part[0],
                                                             g.bias[0], *resln, a.m, g.n[0], n_split)
                : launch_rows<AddLnChosen, zwg_ew::kNormLayer>(g.n[0], a.m, ctx->stream, (const float *)g.part[0],
                                                               g.bias[0], *resln, a.m, g.n[0], n_split);
        if (e != hipSuccess) return fail_hip(ctx, "split-sum + residual + norm kernel launch", e);
    } else if (n_split > 1 && pair) {
        const int64_t elems = (int64_t)(m * (uint64_t)g.n[0]);
        const int bs = small_block(elems);
        zwg_lin::linear_split_sum_swiglu_kernel<<<blocks_for(elems, bs), bs, 0, ctx->stream>>>(g, a.m, n_split);
        e = hipGetLastError();
        if (e != hipSuccess) return fail_hip(ctx, "SwiGLU split-sum kernel launch", e);
    } else if (n_split > 1) {
        const int64_t elems = (int64_t)(m * n_tot);
        const int bs = small_block(elems);
        zwg_lin::linear_split_sum_group_kernel<<<blocks_for(elems, bs), bs, 0, ctx->stream>>>(
            g, a.m, n_split, a.epi);
        e = hipGetLastError();
        if (e != hipSuccess) return fail_hip(ctx, "linear split-sum kernel launch", e);
    }
    return ZWG_OK;
}

int run_q8_stream(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const int8_t *q, const float *scales,
                  const float *bias, uint64_t n, float *out, uint32_t epi) {
    zwg_lin::Q8Args a{};
    a.epi = epi;
    a.x = x;
    a.q = q;
    a.scales = scales;
    a.bias = bias;
    a.out = out;
    a.m = (int32_t)m;
    a.n = (int32_t)n;
    a.k = (int32_t)k;
    a.nb = (int32_t)(k / zwg_lin::kQ8Block);
    return m > 32 ? run_q8_stream_mt<2>(ctx, a) : run_q8_stream_mt<1>(ctx, a);
}

int run_linear(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
               const float *scales, const float *bias, uint64_t n, float *out, uint64_t ldo = 0, uint32_t epi = 0) {
    if (ldo == 0) ldo = n;
    const std::string msg = check_linear(m, k, w_type, n);
    if (ldo < n || ldo > 0x7fffffffull) return fail(ctx, "output row stride must be >= n");
    if (epi > zwg_ew::kEpiAdd) return fail(ctx, "unknown epilogue");
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0 || n == 0) return ZWG_OK;
    if (!x || !w || !out || (w_type == ZWG_W_Q8 && !scales)) return fail(ctx, "null x, w, scales or out");
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(x) || !al16(w) || !al16(out)) return fail(ctx, "x, w and out must be 16-byte aligned");
    if (scales && (reinterpret_cast<uintptr_t>(scales) & 3u)) return fail(ctx, "scales must be 4-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    if (w_type == ZWG_W_Q8 && m <= 64) {
        if (ldo != n) return fail(ctx, "int8 token-step calls write dense rows (output stride n)");
        return run_q8_stream(ctx, x, m, k, static_cast<const int8_t *>(w), scales, bias, n, out, epi);
    }
    LinearArgs a{};
    a.x = x;
    a.w = w;
    a.scales = scales;
    a.bias = bias;
    a.out = out;
    a.ldx = (int64_t)k;
    a.ldw = (int64_t)k;
    a.ldo = (int64_t)ldo;
    a.m = (int32_t)m;
    a.n = (int32_t)n;
    a.k = (int32_t)k;
    a.nb = (int32_t)(k / 32);
    a.epi = epi;
    return w_type == ZWG_W_Q8 ? run_tiled<zwg_lin::kWQ8>(ctx, a) : run_tiled<zwg_lin::kWF16>(ctx, a);
}

} // namespace

int zwg_host::linear_f16_image(zwg_ctx *ctx, const float *x, uint64_t rows, uint64_t k, const void *w,
                               const float *bias, uint64_t n, void *img, int kind, uint64_t n_ctx, uint64_t d) {
    const std::string msg = check_linear(rows, k, ZWG_W_F16, n);
    if (!msg.empty()) return fail(ctx, msg);
    if (kind != 1 && kind != 2) return fail(ctx, "image kind must be 1 (K) or 2 (V)");
    if ((d != 64 && d != 128) || n % d || n_ctx == 0 || n_ctx % 4 || rows % n_ctx)
        return fail(ctx, "tile images need head dim 64 or 128, n a multiple of it and whole items of n_ctx % 4 == 0 keys");
    if (rows == 0) return ZWG_OK;
    const uint64_t tiles_per = (n_ctx + 31) / 32;
    if ((rows / n_ctx) * (n / d) * tiles_per * 64 * d > 0x7fffffffffffull) return fail(ctx, "images too large");
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!x || !w || !img) return fail(ctx, "null x, w or image");
    if (!al16(x) || !al16(w) || !al16(img)) return fail(ctx, "x, w and the image must be 16-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    LinearArgs a{};
    a.x = x;
    a.w = w;
    a.bias = bias;
    a.ldx = (int64_t)k;
    a.ldw = (int64_t)k;
    a.m = (int32_t)rows;
    a.n = (int32_t)n;
    a.k = (int32_t)k;
    a.nb = (int32_t)(k / 32);
    a.img = static_cast<_Float16 *>(img);
    a.img_kind = kind;
    a.img_ctx = (int32_t)n_ctx;
    a.img_d = (int32_t)d;
    a.img_heads = (int32_t)(n / d);
    a.img_tiles = (int32_t)tiles_per;
    a.k_split = (int32_t)k; // never split: the image epilogue is the unsplit kernel's
    const TileChoice tc = choose_tile<zwg_lin::kWF16>(rows, n);
    e = launch_tiled<zwg_lin::kWF16>(a, tc, 1, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "linear (image) kernel launch", e);
    return ZWG_OK;
}

namespace {

// Host-pointer form: stages x (slot 0), the weights (slot 1), the scales and bias (slot 2) and
// out (slot 3) through the context, then waits.
int run_linear_host(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
                    const float *scales, const float *bias, uint64_t n, float *out) {
    const std::string msg = check_linear(m, k, w_type, n);
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0 || n == 0) return ZWG_OK;
    if (!x || !w || !out || (w_type == ZWG_W_Q8 && !scales)) return fail(ctx, "null x, w, scales or out");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    const uint64_t xb = m * k * 4, wb = n * k * (w_type == ZWG_W_Q8 ? 1 : 2);
    const uint64_t sb = w_type == ZWG_W_Q8 ? n * (k / 32) * 4 : 0;
    const uint64_t sb_al = (sb + 15) / 16 * 16, bb = bias ? n * 4 : 0, ob = m * n * 4;
    if (ensure_stage(ctx, 0, xb) || ensure_stage(ctx, 1, wb) || ensure_stage(ctx, 2, sb_al + bb + 16) ||
        ensure_stage(ctx, 3, ob))
        return ZWG_ERROR;
    float *d_scales = sb ? ctx->stage[2] : nullptr;
    float *d_bias = bias ? reinterpret_cast<float *>(reinterpret_cast<char *>(ctx->stage[2]) + sb_al) : nullptr;
    e = hipMemcpyAsync(ctx->stage[0], x, xb, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(ctx->stage[1], w, wb, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && sb) e = hipMemcpyAsync(d_scales, scales, sb, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && bias) e = hipMemcpyAsync(d_bias, bias, bb, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "hipMemcpyAsync (linear upload)", e);
    int rc = run_linear(ctx, ctx->stage[0], m, k, ctx->stage[1], w_type, d_scales, d_bias, n, ctx->stage[3]);
    if (rc != ZWG_OK) return rc;
    e = hipMemcpyAsync(out, ctx->stage[3], ob, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail_hip(ctx, "linear download", e);
    return ZWG_OK;
}

} // namespace

// Device-resident int8 block weights in the packed layout of linear_q8_kernel.hpp (Q8Packed).
struct zwg_q8w {
    zwg_ctx *ctx = nullptr;
    uint64_t n = 0, k = 0;
    int32_t n_slabs = 0, n_chunks = 0;
    uint8_t *q = nullptr;
    float *scales = nullptr;
};

namespace {

const char *const kQ8wClosed = "the int8 weights' context is closed";

// Free the packed weights' device memory (after the work queued on their context's stream).
void free_q8w(zwg_q8w *w) {
    (void)hipSetDevice(w->ctx->device);
    (void)hipStreamSynchronize(w->ctx->stream);
    if (w->q) (void)hipFree(w->q);
    if (w->scales) (void)hipFree(w->scales);
    w->q = nullptr;
    w->scales = nullptr;
}

// zwg_close of the weights' context: the packed copy goes with it
void detach_q8w(void *obj) {
    auto *w = static_cast<zwg_q8w *>(obj);
    free_q8w(w);
    w->ctx = nullptr;
}

// The token-step path (m <= 64) over n_w resident weight sets sharing x and k (checked by the
// callers).
int run_q8w_token_step(zwg_ctx *ctx, const float *x, uint64_t m, uint32_t n_w, const zwg_q8w *const *w,
                       const float *const *bias, float *const *out, uint32_t epi,
                       const zwg_lin::Q8KvStore *kvs = nullptr, const zwg_lin::Q8ResLn *resln = nullptr,
                       Q8PartsOut *po = nullptr, const _Float16 *xcvt_in = nullptr, bool swiglu = false) {
    zwg_lin::Q8Args a{};
    a.x = x;
    a.m = (int32_t)m;
    a.k = (int32_t)w[0]->k;
    a.nb = (int32_t)(w[0]->k / zwg_lin::kQ8Block);
    a.epi = epi;
    zwg_lin::Q8Group g{};
    g.count = (int32_t)n_w;
    g.swiglu = swiglu ? 1 : 0;
    for (uint32_t j = 0; j < n_w; ++j) {
        g.q[j] = w[j]->q;
        g.scales[j] = w[j]->scales;
        g.n_slabs[j] = w[j]->n_slabs;
        g.n[j] = (int32_t)w[j]->n;
        g.bias[j] = bias ? bias[j] : nullptr;
        g.out[j] = out ? out[j] : nullptr;
    }
    return m > 32 ? run_q8p_group<2>(ctx, a, g, kvs, resln, po, xcvt_in)
                  : run_q8p_group<1>(ctx, a, g, kvs, resln, po, xcvt_in);
}

int run_linear_q8w(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, const float *bias, float *out,
                   uint32_t epi) {
    if (!w) return fail(ctx, "null weights");
    if (!w->ctx) return fail(ctx, kQ8wClosed);
    if (epi > zwg_ew::kEpiAdd) return fail(ctx, "unknown epilogue");
    const std::string msg = check_linear(m, w->k, ZWG_W_Q8, w->n);
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0) return ZWG_OK;
    if (!x || !out) return fail(ctx, "null x or out");
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!al16(x) || !al16(out)) return fail(ctx, "x and out must be 16-byte aligned");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    if (m <= ZWG_Q8P_STREAM_ROWS) return run_q8w_token_step(ctx, x, m, 1, &w, &bias, &out, epi);
    LinearArgs a{};
    a.x = x;
    a.w = w->q;
    a.scales = w->scales;
    a.p_chunks = w->n_chunks;
    a.bias = bias;
    a.out = out;
    a.ldx = (int64_t)w->k;
    a.ldo = (int64_t)w->n;
    a.m = (int32_t)m;
    a.n = (int32_t)w->n;
    a.k = (int32_t)w->k;
    a.nb = (int32_t)(w->k / 32);
    a.epi = epi;
    return run_tiled<zwg_lin::kWQ8P>(ctx, a);
}

} // namespace

int zwg_host::linear_q8w_qkv_kv(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *const *w,
                                const float *const *bias, float *q_out, zwg_kv *kv, uint64_t layer, uint64_t seq0,
                                const int32_t *pos_dev, int32_t *n_kv_out, int64_t pos0) {
    if (!ctx) return fail(nullptr, "null context");
    if (!w || !kv) return fail(ctx, "null weight array or cache");
    if (kv->ctx != ctx) return fail(ctx, "the cache belongs to another context (or its context is closed)");
    const zwg_kv_desc &d = kv->desc;
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    for (int j = 0; j < 3; ++j) {
        if (!w[j]) return fail(ctx, "null weights");
        if (!w[j]->ctx) return fail(ctx, kQ8wClosed);
        if (w[j]->k != w[0]->k) return fail(ctx, "q, k and v weights must share k");
        const std::string msg = check_linear(m, w[j]->k, ZWG_W_Q8, w[j]->n);
        if (!msg.empty()) return fail(ctx, msg);
        if (bias && bias[j] && !al16(bias[j])) return fail(ctx, "biases must be 16-byte aligned");
    }
    if (w[1]->n != kv->kvw || w[2]->n != kv->kvw) return fail(ctx, "k and v weights must have n_head_kv * d rows");
    if (w[0]->n % d.d || (w[0]->n / d.d) % d.n_head_kv) return fail(ctx, "q weights must have n_head * d rows, n_head a multiple of n_head_kv");
    if (layer >= d.n_layer) return fail(ctx, "kv layer out of range");
    const bool rows = pos_dev == nullptr; // one sequence's m tokens at pos0 ..
    if (!rows && m > 64) return fail(ctx, "the cache-writing q/k/v call takes at most 64 tokens (one decode step)");
    if (!rows && seq0 + m > d.n_seq) return fail(ctx, "kv sequences out of range");
    if (rows && (seq0 >= d.n_seq || pos0 < 0 || (uint64_t)pos0 + m > d.n_ctx))
        return fail(ctx, "kv sequence out of range, or pos0 + m past the cache");
    if (rows && m > ZWG_Q8P_STREAM_ROWS) return fail(ctx, "one sequence's cache-writing q/k/v call takes at most 256 tokens");
    if (m == 0) return ZWG_OK;
    if (!x || !al16(x) || !q_out || !al16(q_out)) return fail(ctx, "x and q_out must be non-null and 16-byte aligned");
    const hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    zwg_lin::Q8KvStore kvs{};
    kvs.q_out = q_out;
    kvs.k_cache = kv->k + layer * d.n_seq * kv->per_seq;
    kvs.v_cache = kv->v + layer * d.n_seq * kv->per_seq;
    kvs.cos = kv->cos;
    kvs.sin = kv->sin;
    kvs.pos_dev = pos_dev;
    kvs.n_kv_out = n_kv_out;
    kvs.per_seq = (int64_t)kv->per_seq;
    kvs.seq0 = (int32_t)seq0;
    kvs.n_ctx = (int32_t)d.n_ctx;
    kvs.n_head = (int32_t)(w[0]->n / d.d);
    kvs.n_head_kv = (int32_t)d.n_head_kv;
    kvs.kt = d.layout == ZWG_KV_KT;
    kvs.d = (int32_t)d.d;
    kvs.pos0 = rows ? (int32_t)pos0 : 0;
    kvs.seq_step = rows ? 0 : 1;
    return run_q8w_token_step(ctx, x, m, 3, w, bias, nullptr, zwg_ew::kEpiNone, &kvs);
}

// x += xin . W^T + bias and ln_out = the norm of x (layer norm with ln_w, ln_b, or RMS norm with
// ln_w; eps) for a decode step's or a prompt batch's rows (m <= 256, n <= 4096): one stream launch and
// linear_split_sum_add_ln_kernel; a call too short to split k (k <= 256) runs the add epilogue and
// the norm as two launches, with the same results.  xcvt_out (33..64 rows): ln_out also split for
// the next call (q8w_xcvt_halves(n) halves), which takes it as xcvt_in.
int zwg_host::linear_q8w_add_ln(zwg_ctx *ctx, const float *xin, uint64_t m, const zwg_q8w *w, const float *bias,
                                float *x, const float *ln_w, const float *ln_b, float eps, float *ln_out, int norm,
                                _Float16 *xcvt_out) {
    if (!w || !w->ctx) return fail(ctx, w ? kQ8wClosed : "null weights");
    const std::string msg = check_linear(m, w->k, ZWG_W_Q8, w->n);
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0) return ZWG_OK;
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (m > ZWG_Q8P_STREAM_ROWS || w->n % 4 || w->n > (uint64_t)kMaxRowN)
        return fail(ctx, "the fused residual + norm call takes m <= 256 and n <= 4096, n % 4 == 0");
    const bool rms = norm == zwg_ew::kNormRms;
    if (!xin || !x || !ln_w || (!rms && !ln_b) || !ln_out || !al16(xin) || !al16(x) || !al16(ln_w) ||
        (ln_b && !al16(ln_b)) || !al16(ln_out) || (bias && !al16(bias)))
        return fail(ctx, "null or unaligned buffer (all 16-byte aligned)");
    if (xcvt_out && (m <= 32 || !al16(xcvt_out)))
        return fail(ctx, "split rows for the next call are for 33..64-row steps (16-byte aligned)");
    if (w->n_chunks < 2) {
        if (xcvt_out) return fail(ctx, "the split rows for the next call need k above 256");
        const int rc = run_linear_q8w(ctx, xin, m, w, bias, x, zwg_ew::kEpiAdd);
        if (rc != ZWG_OK) return rc;
        return rms ? rms_norm(ctx, x, m, w->n, ln_w, eps, ln_out) : layer_norm(ctx, x, m, w->n, ln_w, ln_b, eps, ln_out);
    }
    zwg_lin::Q8ResLn r{x, ln_w, ln_b, ln_out, eps, rms ? zwg_ew::kNormRms : zwg_ew::kNormLayer, xcvt_out};
    float *outs[1] = {x};
    return run_q8w_token_step(ctx, xin, m, 1, &w, &bias, outs, zwg_ew::kEpiAdd, nullptr, &r);
}

bool zwg_host::q8w_group_reads_xcvt(uint64_t m, uint32_t n_w, const zwg_q8w *const *w) {
    if (m <= 32 || m > 64 || n_w == 0 || n_w > (uint32_t)zwg_lin::kQ8MaxGroup) return false;
    constexpr int kRows = 32 * q8p_waves<2>();
    int64_t gx = 0;
    for (uint32_t j = 0; j < n_w; ++j) gx += ((int64_t)w[j]->n + kRows - 1) / kRows;
    const int n_chunks = (int)((w[0]->k + zwg_lin::kQ8Chunk - 1) / zwg_lin::kQ8Chunk);
    return !q8p_splits_x_itself<2>(gx, n_chunks);
}

uint64_t zwg_host::q8w_stream_rows() { return ZWG_Q8P_STREAM_ROWS; }

// out = silu(x . gate^T) * (x . up^T) for at most q8w_stream_rows() rows (src/llm.zig:207-210):
// one stream launch over both weight sets (a SwiGLU pair), plus one SwiGLU split sum when k is
// split; the same values as the two projections' group call followed by the SiLU-mul kernel.
// xcvt_in as for linear_q8w_group_xcvt.
int zwg_host::linear_q8w_swiglu(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *gate, const zwg_q8w *up,
                                float *out, const _Float16 *xcvt_in) {
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!gate || !up) return fail(ctx, "null weights");
    if (!gate->ctx || !up->ctx) return fail(ctx, kQ8wClosed);
    if (gate->n != up->n || gate->k != up->k) return fail(ctx, "gate and up weights must have one shape");
    const std::string msg = check_linear(m, gate->k, ZWG_W_Q8, gate->n);
    if (!msg.empty()) return fail(ctx, msg);
    if (m == 0) return ZWG_OK;
    if (m > ZWG_Q8P_STREAM_ROWS || !x || !out || !al16(x) || !al16(out) ||
        (xcvt_in && (!al16(xcvt_in) || m <= 32 || m > 64)))
        return fail(ctx, "a SwiGLU call: m <= 256, x and out 16-byte aligned, split rows for 33..64 rows");
    const zwg_q8w *w[2] = {gate, up};
    float *outs[2] = {out, nullptr};
    return run_q8w_token_step(ctx, x, m, 2, w, nullptr, outs, zwg_ew::kEpiNone, nullptr, nullptr, nullptr, xcvt_in,
                              true);
}

uint64_t zwg_host::q8w_xcvt_halves(uint64_t k) {
    return (k + zwg_lin::kQ8Chunk - 1) / zwg_lin::kQ8Chunk * (uint64_t)zwg_lin::q8_chunk_halves<2>();
}

// A grouped token-step call (as zwg_linear_q8w_group_dev, m <= 64) whose x was split by the
// previous call (linear_q8w_add_ln's xcvt_out, from the same rows); used where the call streams
// its x from a split pass (33..64 rows, unsplit k), ignored where it splits x itself.
int zwg_host::linear_q8w_group_xcvt(zwg_ctx *ctx, const float *x, uint64_t m, uint32_t n_w, const zwg_q8w *const *w,
                                    const float *const *bias, float *const *out, const _Float16 *xcvt_in) {
    if (n_w == 0 || n_w > (uint32_t)zwg_lin::kQ8MaxGroup || !w || !out) return fail(ctx, "n_w must be 1..4");
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    for (uint32_t j = 0; j < n_w; ++j) {
        if (!w[j] || !w[j]->ctx) return fail(ctx, w[j] ? kQ8wClosed : "null weights");
        if (w[j]->k != w[0]->k) return fail(ctx, "the weights of a group must share k");
        const std::string msg = check_linear(m, w[j]->k, ZWG_W_Q8, w[j]->n);
        if (!msg.empty()) return fail(ctx, msg);
        if (m && (!out[j] || !al16(out[j]))) return fail(ctx, "outputs must be non-null and 16-byte aligned");
    }
    if (m == 0) return ZWG_OK;
    if (m > 64 || !x || !al16(x) || (xcvt_in && (!al16(xcvt_in) || m <= 32)))
        return fail(ctx, "a token-step group call: m <= 64, x 16-byte aligned, split rows for 33..64 rows");
    return run_q8w_token_step(ctx, x, m, n_w, w, bias, out, zwg_ew::kEpiNone, nullptr, nullptr, nullptr, xcvt_in);
}

int zwg_host::linear_q8w_parts(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, float *parts,
                               int max_parts, int *n_split) {
    if (!w || !w->ctx) return fail(ctx, w ? kQ8wClosed : "null weights");
    const std::string msg = check_linear(m, w->k, ZWG_W_Q8, w->n);
    if (!msg.empty()) return fail(ctx, msg);
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (m == 0 || m > 64 || w->n_chunks < 2 || max_parts < 2 || w->n % 4)
        return fail(ctx, "projection partials: 1 <= m <= 64, k above 256, n % 4 == 0, room for two splits");
    if (!x || !parts || !n_split || !al16(x) || !al16(parts)) return fail(ctx, "null or unaligned buffer");
    Q8PartsOut po{parts, max_parts, 0};
    const int rc = run_q8w_token_step(ctx, x, m, 1, &w, nullptr, nullptr, zwg_ew::kEpiNone, nullptr, nullptr, &po);
    *n_split = po.n_split;
    return rc;
}

// x[i] = te.row(tok[i]) + pe[pos[i]] and ln_out[i] = the norm of x[i] (q8p_embed_ln_kernel).
int zwg_host::q8w_embed_ln(zwg_ctx *ctx, const zwg_q8w *te, const int32_t *tok, const float *pe, const int32_t *pos,
                           uint64_t pe_rows, uint64_t m, float *x, const float *ln_w, const float *ln_b, float eps,
                           float *ln_out, int norm) {
    if (!te || !te->ctx) return fail(ctx, te ? kQ8wClosed : "null weights");
    if (m == 0) return ZWG_OK;
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (te->k % 4 || te->k > (uint64_t)kMaxRowN || m > 0x7fffffffull || pe_rows > 0x7fffffffull)
        return fail(ctx, "embedding rows of at most 4096 floats, a multiple of 4");
    const bool rms = norm == zwg_ew::kNormRms;
    if (!tok || !x || !ln_w || (!rms && !ln_b) || !ln_out || (pe_rows && (!pe || !pos)) || !al16(x) || !al16(ln_w) ||
        (ln_b && !al16(ln_b)) || !al16(ln_out) || (pe && !al16(pe)))
        return fail(ctx, "null or unaligned buffer (all 16-byte aligned)");
    zwg_lin::Q8Packed tp{te->q, te->scales, te->n_slabs, te->n_chunks};
    zwg_lin::Q8ResLn r{nullptr, ln_w, ln_b, ln_out, eps, rms ? zwg_ew::kNormRms : zwg_ew::kNormLayer};
    const hipError_t e =
        rms ? launch_rows<EmbedLnRows, zwg_ew::kNormRms>((int32_t)te->k, (int32_t)m, ctx->stream, tp, (int32_t)te->n,
                                                         tok, pe, pos, (int32_t)pe_rows, (int32_t)m, (int32_t)te->k, x, r)
            : launch_rows<EmbedLnRows, zwg_ew::kNormLayer>((int32_t)te->k, (int32_t)m, ctx->stream, tp,
                                                           (int32_t)te->n, tok, pe, pos, (int32_t)pe_rows, (int32_t)m,
                                                           (int32_t)te->k, x, r);
    return e == hipSuccess ? ZWG_OK : fail_hip(ctx, "token embedding kernel launch", e);
}

extern "C" {

int zwg_q8w_create(zwg_ctx *ctx, const int8_t *q, const float *scales, uint64_t n, uint64_t k, uint32_t flags,
                   zwg_q8w **out) {
    if (out) *out = nullptr;
    if (!ctx || !out) return fail(ctx, "null context or out");
    const std::string msg = check_linear(1, k, ZWG_W_Q8, n);
    if (!msg.empty()) return fail(ctx, msg);
    if (n == 0 || !q || !scales) return fail(ctx, "empty matrix or null q / scales");
    if (flags & ~ZWG_Q8W_FROM_HOST) return fail(ctx, "unknown flags");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    auto *w = new zwg_q8w();
    w->ctx = ctx;
    w->n = n;
    w->k = k;
    w->n_slabs = (int32_t)((n + 31) / 32);
    w->n_chunks = (int32_t)((k + zwg_lin::kQ8Chunk - 1) / zwg_lin::kQ8Chunk);
    const int64_t qb = zwg_lin::q8p_q_bytes(w->n_slabs, w->n_chunks);
    const int64_t sb = zwg_lin::q8p_scale_bytes(w->n_slabs, w->n_chunks);
    void *pq = nullptr, *ps = nullptr;
    e = hipMalloc(&pq, (size_t)qb);
    if (e == hipSuccess) e = hipMalloc(&ps, (size_t)sb);
    if (e != hipSuccess) {
        if (pq) (void)hipFree(pq);
        delete w;
        return fail_hip(ctx, "hipMalloc (int8 weights)", e);
    }
    w->q = static_cast<uint8_t *>(pq);
    w->scales = static_cast<float *>(ps);
    const int8_t *src_q = q;
    const float *src_s = scales;
    void *tq = nullptr, *ts = nullptr;
    if (flags & ZWG_Q8W_FROM_HOST) { // stage the raw arrays, pack on the device, free the staging
        e = hipMalloc(&tq, (size_t)(n * k));
        if (e == hipSuccess) e = hipMalloc(&ts, (size_t)(n * (k / 32) * 4));
        if (e == hipSuccess) e = hipMemcpyAsync(tq, q, n * k, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(ts, scales, n * (k / 32) * 4, hipMemcpyHostToDevice, ctx->stream);
        src_q = static_cast<const int8_t *>(tq);
        src_s = static_cast<const float *>(ts);
    } else if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(scales) & 3u)) {
        e = hipErrorInvalidValue;
    }
    if (e == hipSuccess) {
        zwg_lin::linear_q8_pack_kernel<<<2048, 256, 0, ctx->stream>>>(src_q, src_s, (int32_t)n, (int32_t)k, w->q,
                                                                     w->scales, w->n_slabs, w->n_chunks);
        e = hipGetLastError();
    }
    if (e == hipSuccess && (flags & ZWG_Q8W_FROM_HOST)) e = hipStreamSynchronize(ctx->stream);
    if (tq) (void)hipFree(tq);
    if (ts) (void)hipFree(ts);
    if (e != hipSuccess) {
        (void)hipFree(w->q);
        (void)hipFree(w->scales);
        delete w;
        return fail_hip(ctx, "int8 weight packing (q 16-byte and scales 4-byte aligned?)", e);
    }
    add_child(ctx, w, detach_q8w);
    *out = w;
    return ZWG_OK;
}

void zwg_q8w_destroy(zwg_q8w *w) {
    if (!w) return;
    if (w->ctx) {
        remove_child(w->ctx, w);
        free_q8w(w);
    }
    delete w;
}

int zwg_q8w_shape(const zwg_q8w *w, uint64_t *n, uint64_t *k) {
    if (w && !w->ctx) return fail(nullptr, kQ8wClosed);
    if (!w) return fail(nullptr, "null weights");
    if (n) *n = w->n;
    if (k) *k = w->k;
    return ZWG_OK;
}

int zwg_linear_q8w_dev(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, const float *bias, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    return run_linear_q8w(ctx, x, m, w, bias, out, zwg_ew::kEpiNone);
}

int zwg_linear_q8w_epi_dev(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *w, const float *bias, float *out,
                           uint32_t epilogue) {
    if (!ctx) return fail(nullptr, "null context");
    return run_linear_q8w(ctx, x, m, w, bias, out, epilogue);
}

int zwg_linear_q8w_group_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint32_t n_w, const zwg_q8w *const *w,
                             const float *const *bias, float *const *out) {
    if (!ctx) return fail(nullptr, "null context");
    if (n_w == 0 || n_w > (uint32_t)zwg_lin::kQ8MaxGroup) return fail(ctx, "n_w must be 1..4");
    if (!w || !out) return fail(ctx, "null weight or output array");
    const auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    for (uint32_t j = 0; j < n_w; ++j) {
        if (!w[j]) return fail(ctx, "null weights");
        if (!w[j]->ctx) return fail(ctx, kQ8wClosed);
        if (w[j]->k != w[0]->k) return fail(ctx, "the weights of a group must share k");
        const std::string msg = check_linear(m, w[j]->k, ZWG_W_Q8, w[j]->n);
        if (!msg.empty()) return fail(ctx, msg);
        if (m && (!out[j] || !al16(out[j]))) return fail(ctx, "outputs must be non-null and 16-byte aligned");
    }
    if (m == 0) return ZWG_OK;
    if (!x || !al16(x)) return fail(ctx, "x must be non-null and 16-byte aligned");
    if (m > ZWG_Q8P_STREAM_ROWS) { // prefill sizes: the tiled kernel, one call per set
        for (uint32_t j = 0; j < n_w; ++j) {
            const int r = run_linear_q8w(ctx, x, m, w[j], bias ? bias[j] : nullptr, out[j], zwg_ew::kEpiNone);
            if (r != ZWG_OK) return r;
        }
        return ZWG_OK;
    }
    const hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return fail_hip(ctx, "hipSetDevice", e);
    return run_q8w_token_step(ctx, x, m, n_w, w, bias, out, zwg_ew::kEpiNone);
}

int zwg_linear_q8w_qkv_kv_dev(zwg_ctx *ctx, const float *x, uint64_t m, const zwg_q8w *const *w,
                              const float *const *bias, float *q_out, zwg_kv *kv, uint64_t layer, uint64_t seq0,
                              const int32_t *pos_dev) {
    if (!ctx) return fail(nullptr, "null context");
    if (!pos_dev) return fail(ctx, "null pos_dev");
    return linear_q8w_qkv_kv(ctx, x, m, w, bias, q_out, kv, layer, seq0, pos_dev, nullptr);
}

int zwg_linear_epi_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
                       const float *bias, uint64_t n, float *out, uint64_t out_stride, uint32_t epilogue) {
    if (!ctx) return fail(nullptr, "null context");
    if (w_type != ZWG_W_F16) return fail(ctx, "zwg_linear_epi_dev takes ZWG_W_F16 weights (zwg_linear_q8w_epi_dev: int8)");
    return run_linear(ctx, x, m, k, w, w_type, nullptr, bias, n, out, out_stride, epilogue);
}


int zwg_linear_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
                   const float *bias, uint64_t n, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    if (w_type != ZWG_W_F16) return fail(ctx, "zwg_linear_dev takes ZWG_W_F16 weights (zwg_linear_q8_dev: int8)");
    return run_linear(ctx, x, m, k, w, w_type, nullptr, bias, n, out);
}

int zwg_linear(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const void *w, uint32_t w_type,
               const float *bias, uint64_t n, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    if (w_type != ZWG_W_F16) return fail(ctx, "zwg_linear takes ZWG_W_F16 weights (zwg_linear_q8: int8)");
    return run_linear_host(ctx, x, m, k, w, w_type, nullptr, bias, n, out);
}

int zwg_linear_q8_dev(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const int8_t *q, const float *scales,
                      const float *bias, uint64_t n, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    return run_linear(ctx, x, m, k, q, ZWG_W_Q8, scales, bias, n, out);
}

int zwg_linear_q8(zwg_ctx *ctx, const float *x, uint64_t m, uint64_t k, const int8_t *q, const float *scales,
                  const float *bias, uint64_t n, float *out) {
    if (!ctx) return fail(nullptr, "null context");
    return run_linear_host(ctx, x, m, k, q, ZWG_W_Q8, scales, bias, n, out);
}

} // extern "C"
