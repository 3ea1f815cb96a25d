// Linear layers over int8 block weights on gfx950 MFMA: ops.linear with a gemm.Q8
// (src/ops.zig:283-306, src/gemm.zig:188-351).  q int8 [n][k], scales f32 [n][k / 32]:
//
//     out[i][o] = sum_b scales[o][b] * (sum_{p in block b} x[i][p] * q[o][p])  (+ bias[o])
//
// with blocks of 32 along k, each block's partial dot product scaled once (gemm.dotQ,
// src/gemm.zig:274-286, and micro4x4Q, :289-327, do the same per vector lane).
//
// Precision.  An int8 weight is exact in f16.  Each f32 activation is split into two f16 terms,
// x = hi + lo (hi = f16(x), lo = f16(x - hi)), which keep 22 of x's 24 significand bits; a
// block's two MFMAs per term accumulate hi*q and lo*q in f32, and the block sum is scaled in f32
// on the VALU.  |x| must stay within f16's range (65504).
//
// Two kernels:
//
// * linear_q8_stream_kernel<MT, S>: m <= 64 (decoder and LLM token steps, logits).  The weights
//   are the stream: every int8 byte is read from HBM once, 16 bytes per lane per load (one Q8
//   block of 32 weight rows per wave-load).  A workgroup of 4 waves owns 4*S slabs of 32 weight
//   rows and walks k in chunks of 256 (8 blocks).  x is split into hi/lo halves once per call by
//   linear_q8_xprep_kernel, in the exact order the MFMA A operand wants it; each workgroup copies
//   a chunk of it into LDS with direct global-to-LDS loads (no VGPRs, no VALU), issued before the
//   chunk's weight loads so the wait for x never waits on the weights.  An operand read is then
//   1 KB contiguous per wave (conflict-free ds_read_b128).
//   v_mfma_f32_32x32x16_f16 with A = x rows, B = weight rows: lane l's 16 weight bytes
//   q[row l%32][kb + 16 (l/32) .. +16] feed the block's two k-steps (bytes 0-7, then 8-15), and
//   the result column l%32 is the weight row, so the block's scale is one f32 per lane.
//   When the weight rows alone give too few workgroups to fill the chip, k is split over
//   gridDim.y and linear_split_sum_kernel adds the partial sums in a fixed order.
//
// * linear_mfma_kernel<BM, BN, true> (linear_kernel.hpp): larger m, the tiled GEMM with the
//   weight tile widened to f16 on its way into LDS and the same per-block scaling.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16, measured on the device): lane l, half s of A is
// A[l % 32][8 (l / 32) + s], of B is B[8 (l / 32) + s][l % 32]; result register r of lane l is
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <type_traits>

#include "linear_kernel.hpp"

namespace zwg_lin {

constexpr int kQ8Block = 32;                // src/gemm.zig:194
constexpr int kQ8Chunk = 256;               // k per LDS chunk of the stream kernel
constexpr int kQ8ChunkBlocks = kQ8Chunk / kQ8Block;
constexpr int kQ8Threads = 256;
// The packed weights and scales are read once per call: non-temporal loads (cache policy nt)
// stream them past the caches, which keep the x stages every workgroup reuses.
constexpr int kQ8CachePolicyNT = 2;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
__host__ __device__ constexpr int q8_vmcnt(int n) {
    return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8);
}

struct Q8Args {
    const float *x;      // [m][k]
    const int8_t *q;     // [n][k]
    const float *scales; // [n][nb]
    const float *bias;   // [n] or nullptr
    float *out;          // [m][n]
    float *part;         // [n_split][m][n] when n_split > 1
    int32_t m, n, k, nb;
    int32_t chunks_per_split, n_split;
    uint32_t epi; // zwg_ew::kEpi*, applied where `out` is written (here, or by the split sum)
};

// Layout of x's hi/lo halves, per chunk of 256 k: [block][m-tile][hi/lo][k-step][lane][8 halves],
// 32 KB per m-tile.  Lane l, k-step s of (block b, m-tile i) holds x[32 i + l % 32][kb + 16 (l / 32)
// + 8 s + 0..7], kb = 32 b.  One [hi/lo][k-step] piece of a (block, m-tile) is 1 KB: 64 lanes x 16 B.
template <int MT>
__host__ __device__ constexpr int q8_chunk_halves() {
    return kQ8ChunkBlocks * MT * 2 * 2 * 64 * 8;
}
template <int MT>
__device__ __forceinline__ int q8_xs_at(int b, int i, int hl, int s, int lane) {
    return ((((b * MT + i) * 2 + hl) * 2 + s) * 64 + lane) * 8;
}

// x[row][gk .. gk + 3] (gk % 4 == 0) split into f16 hi/lo halves at its place in xcvt's chunk
// layout above: hi = f16(v), lo = f16(v - hi)
template <int MT>
__device__ __forceinline__ void q8_xs_store(_Float16 *xcvt, int row, int gk, f32x4 v) {
    const int c = gk / kQ8Chunk, kk = gk % kQ8Chunk;
    const int b = kk >> 5, kb = kk & 31;
    const int gg = kb >> 4, s = (kb >> 3) & 1, j = kb & 7;
    const int i = row >> 5, l = (row & 31) + 32 * gg;
    half4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        hi[e] = (_Float16)v[e];
        lo[e] = (_Float16)(v[e] - (float)hi[e]);
    }
    _Float16 *base = xcvt + (int64_t)c * q8_chunk_halves<MT>();
    *reinterpret_cast<half4 *>(base + q8_xs_at<MT>(b, i, 0, s, l) + j) = hi;
    *reinterpret_cast<half4 *>(base + q8_xs_at<MT>(b, i, 1, s, l) + j) = lo;
}

// x f32 [m][k] -> xcvt f16 [n_chunks][chunk layout above]; rows >= m and columns >= k are 0.
// One thread per 4 consecutive k of one row.
template <int MT>
__global__ __launch_bounds__(256) void linear_q8_xprep_kernel(const float *x, _Float16 *xcvt, int32_t m, int32_t k,
                                                             int32_t n_chunks) {
    const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_chunk = MT * 32 * (kQ8Chunk / 4);
    if (f >= per_chunk * n_chunks) return;
    const int c = (int)(f / per_chunk), rem = (int)(f % per_chunk);
    const int row = rem / (kQ8Chunk / 4), kk = 4 * (rem % (kQ8Chunk / 4));
    const int gk = c * kQ8Chunk + kk;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (row < m && gk < k) v = *reinterpret_cast<const f32x4 *>(x + (int64_t)row * k + gk);
    q8_xs_store<MT>(xcvt, row, gk, v);
}

template <int MT, int S>
__global__ __launch_bounds__(kQ8Threads) void linear_q8_stream_kernel(Q8Args a, const _Float16 *xcvt) {
    constexpr int NB = kQ8ChunkBlocks;
    constexpr int ROWS = 4 * S * 32;                   // weight rows per workgroup
    constexpr int PIECES = q8_chunk_halves<MT>() / 512; // 1 KB pieces of an x chunk
    constexpr int XL = PIECES / 4;                      // pieces each wave copies
    __shared__ __align__(16) _Float16 xs[q8_chunk_halves<MT>()];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int n0 = blockIdx.x * ROWS;
    const int wrow0 = wave * S * 32; // this wave's first row within the workgroup's slab group
    const int split = blockIdx.y;
    const int n_chunks = (a.k + kQ8Chunk - 1) / kQ8Chunk;
    const int c_begin = split * a.chunks_per_split;
    const int c_end = min(c_begin + a.chunks_per_split, n_chunks);

    // q / scales: rows past n read as 0.  x_src: the call's prepared x chunks.
    const __amdgpu_buffer_rsrc_t x_src = rsrc(xcvt, (uint32_t)n_chunks * (uint32_t)PIECES * 1024u);
    const int rows_w = min(ROWS, a.n - n0);
    const __amdgpu_buffer_rsrc_t q_src = rsrc(a.q + (int64_t)n0 * a.k, (uint32_t)((int64_t)rows_w * a.k));
    const __amdgpu_buffer_rsrc_t s_src = rsrc(a.scales + (int64_t)n0 * a.nb, (uint32_t)((int64_t)rows_w * a.nb * 4));
    uint32_t qbase[S], sbase[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int row = wrow0 + s * 32 + r32;
        qbase[s] = (uint32_t)(row * a.k + 16 * g);
        sbase[s] = (uint32_t)(row * a.nb) * 4u;
    }

    f32x16 acc[MT][S];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int s = 0; s < S; ++s) acc[i][s] = (f32x16){0};

    for (int c = c_begin; c < c_end; ++c) {
        const int k0 = c * kQ8Chunk;
        __syncthreads(); // the previous chunk's operand reads are done
        // x chunk into LDS: wave w copies pieces w, w + 4, ...; lane l's 16 bytes land at l * 16
#pragma unroll
        for (int u = 0; u < XL; ++u) {
            const int piece = wave + 4 * u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(x_src, (__attribute__((address_space(3))) void *)(xs + piece * 512), 16,
                                                 (uint32_t)((c * PIECES + piece) * 1024 + lane * 16), 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        // This wave's weights for the chunk (slab s, block b: 16 bytes per lane) and the blocks'
        // scales.  A block past k gets scale 0 (its offset is out of range), so whatever the
        // weight load returned there adds exactly nothing.
        u32x4 wq[S][NB];
        float sc[S][NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int kb = k0 + b * kQ8Block;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                wq[s][b] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(q_src, (int)(qbase[s] + (uint32_t)kb), 0, 0));
                const uint32_t soff = kb < a.k ? sbase[s] + (uint32_t)(kb / kQ8Block) * 4u : kOutOfRange;
                sc[s][b] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_src, (int)soff, 0, 0));
            }
        }
        // wait for this wave's x pieces only (loads complete in order; the 2 S NB weight and
        // scale loads were issued after them), then for every wave's
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(q8_vmcnt(2 * S * NB));
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int b = 0; b < NB; ++b) {
            half8 ah[MT][2], al[MT][2];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    ah[i][s] = *reinterpret_cast<const half8 *>(&xs[q8_xs_at<MT>(b, i, 0, s, lane)]);
                    al[i][s] = *reinterpret_cast<const half8 *>(&xs[q8_xs_at<MT>(b, i, 1, s, lane)]);
                }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const half8 w0 = int8x8_to_half8(wq[s][b][0], wq[s][b][1]);
                const half8 w1 = int8x8_to_half8(wq[s][b][2], wq[s][b][3]);
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    f32x16 t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], w0, (f32x16){0}, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], w0, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], w1, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], w1, t, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][s][r] = __builtin_fmaf(t[r], sc[s][b], acc[i][s][r]);
                }
            }
        }
    }

    // register r of lane l: row 32 i + 8 (r / 4) + 4 (l / 32) + r % 4, column (weight row) l % 32
    float *dst = a.n_split > 1 ? a.part + (int64_t)split * a.m * a.n : a.out;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int col = n0 + wrow0 + s * 32 + r32;
        if (col >= a.n) continue;
        const float bj = (a.n_split == 1 && a.bias) ? a.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (row < a.m) {
                    if (a.n_split > 1) dst[(int64_t)row * a.n + col] = acc[i][s][r];
                    else zwg_ew::epilogue_store(&dst[(int64_t)row * a.n + col], acc[i][s][r] + bj, a.epi);
                }
            }
    }
}

// Packed device weights (zwg_q8w): the same int8 and scales, laid out for the stream kernel so
// that every wave-load is contiguous.  n is padded to whole slabs of 32 rows, k to whole chunks
// of 256 (8 blocks); padding is zero (scale 0).
//   q:      [slab][block][lane][16 bytes], lane l of (slab s, block b) holding
//           q[32 s + l % 32][32 b + 16 (l / 32) .. +16]: one 1 KB tile per (slab, block).
//   scales: [slab][chunk][32 rows][8 blocks] f32: a lane's 8 block scales of a chunk are 32
//           contiguous bytes, and the 32 rows of a slab 1 KB.
struct Q8Packed {
    const uint8_t *q;
    const float *scales;
    int32_t n_slabs, n_chunks;
};

// Weight sets of one token-step launch over the same x (a decode step's q/k/v, or gate/up): set j
// takes workgroups block_start[j] .. block_start[j + 1] - 1 of the stream kernel and elements
// elem_start[j] .. elem_start[j + 1] - 1 of the split sum; all sets share x, k and the k split.
constexpr int kQ8MaxGroup = 4;
struct Q8Group {
    int32_t count;
    int32_t n_chunks; // k / 256, rounded up: the same for every set
    int32_t block_start[kQ8MaxGroup + 1];
    int64_t elem_start[kQ8MaxGroup + 1];
    const uint8_t *q[kQ8MaxGroup]; // packed weights of set j (Q8Packed)
    const float *scales[kQ8MaxGroup];
    int32_t n_slabs[kQ8MaxGroup];
    int32_t n[kQ8MaxGroup];
    const float *bias[kQ8MaxGroup];
    float *out[kQ8MaxGroup];
    float *part[kQ8MaxGroup]; // [n_split][m][n[j]] when the call is split
    // 1: a SwiGLU pair (count 2, n[0] == n[1]: the MLP's gate and up, src/llm.zig:207-210): each
    // workgroup takes the same columns of both sets and the call stores silu(gate) * up into
    // out[0] (linear_q8p_stream_kernel; split calls through linear_split_sum_swiglu_kernel)
    int32_t swiglu;
};

// entry j of a group field, by selects on the uniform j (no dynamic indexing of the kernel-
// argument struct, which would go through scratch)
template <typename T, int N>
__device__ __forceinline__ T q8_pick(const T (&v)[N], int j) {
    T r = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) r = j == i ? v[i] : r;
    return r;
}
__device__ __forceinline__ int q8_group_of_block(const Q8Group &g, int bx) {
    int j = 0;
#pragma unroll
    for (int i = 1; i < kQ8MaxGroup; ++i) j += (i < g.count && bx >= g.block_start[i]) ? 1 : 0;
    return j;
}
__device__ __forceinline__ int q8_group_of_elem(const Q8Group &g, int64_t e) {
    int j = 0;
#pragma unroll
    for (int i = 1; i < kQ8MaxGroup; ++i) j += (i < g.count && e >= g.elem_start[i]) ? 1 : 0;
    return j;
}

__host__ __device__ inline int64_t q8p_q_bytes(int64_t n_slabs, int64_t n_chunks) {
    return n_slabs * n_chunks * kQ8ChunkBlocks * 1024;
}
__host__ __device__ inline int64_t q8p_scale_bytes(int64_t n_slabs, int64_t n_chunks) {
    return n_slabs * n_chunks * 32 * kQ8ChunkBlocks * 4;
}

// Pack q [n][k] (int8) and scales [n][k / 32] into the layout above: one thread per 16-byte
// piece of a q tile (and, for the first 8 lanes of a slab's chunk, nothing else); scales by a
// second grid-stride pass in the same kernel.
__global__ __launch_bounds__(256) void linear_q8_pack_kernel(const int8_t *q, const float *scales, int32_t n,
                                                            int32_t k, uint8_t *pq, float *ps, int32_t n_slabs,
                                                            int32_t n_chunks) {
    const int32_t nb = k / kQ8Block, nbp = n_chunks * kQ8ChunkBlocks;
    const int64_t pieces = (int64_t)n_slabs * nbp * 64;
    const int64_t sc_elems = (int64_t)n_slabs * n_chunks * 32 * kQ8ChunkBlocks;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x; f < pieces; f += stride) {
        const int lane = (int)(f & 63);
        const int64_t tile = f >> 6;
        const int b = (int)(tile % nbp);
        const int64_t slab = tile / nbp;
        const int64_t row = slab * 32 + (lane & 31);
        const int kk = b * kQ8Block + 16 * (lane >> 5);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < n && kk < k) v = *reinterpret_cast<const u32x4 *>(q + row * k + kk);
        *reinterpret_cast<u32x4 *>(pq + f * 16) = v;
    }
    for (int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x; f < sc_elems; f += stride) {
        const int b8 = (int)(f & 7);
        const int r = (int)((f >> 3) & 31);
        const int64_t sc_chunk = f >> 8; // slab * n_chunks + chunk
        const int c = (int)(sc_chunk % n_chunks);
        const int64_t slab = sc_chunk / n_chunks;
        const int64_t row = slab * 32 + r;
        const int b = c * kQ8ChunkBlocks + b8;
        ps[f] = (row < n && b < nb) ? scales[row * nb + b] : 0.f;
    }
}

// The stream kernel over packed weights, software-pipelined.  k is walked in stages of 4 blocks
// (128 k).  x stages sit in LDS double-buffered and each wave keeps two register sets of weights
// and scales, so the loads of stage t + 1 (x, then weights, then scales) are in flight while stage
// t's MFMAs run: at the top of stage t the wave waits only for its x of stage t (loads complete in
// order, and stage t's weights were issued after them), and the barrier that follows tells every
// wave that the stage's x is in LDS (and that stage t - 1's buffer is free again).  Two x paths:
//   XS = false: x was split into f16 hi/lo halves in the MFMA A-operand order (q8_xs_at) by
//     linear_q8_xprep_kernel; each stage's pieces are copied into LDS by direct global-to-LDS loads
//     (no VGPRs, no VALU).
//   XS = true: no separate pass.  A stage's f32 x rows arrive in registers (coalesced 16-byte
//     loads) and each workgroup splits them and writes them into the LDS stage itself before the
//     barrier.  This costs registers and a short split before each barrier, and saves a launch:
//     the better trade for 32-row calls and for small 64-row calls whose k is split (measured:
//     Whisper small.en decoder step 784 -> 681 us, Qwen2.5-1.5B decode step 2095 -> 1960 us), the
//     worse one for a large unsplit 64-row call (Qwen2.5-1.5B logits 109 -> 150 us).
// Padding blocks (k is padded to 256) have scale 0 and x 0; a stage wholly past k is not run.
constexpr int kQ8StageBlocks = 4;
constexpr int kQ8StageK = kQ8StageBlocks * kQ8Block;

// KS = 2: the workgroup's waves form two groups of NW, each over the same slabs and half of the
// workgroup's stages (contiguous, each half a whole number of 2-stage turns), with x buffers of
// their own; at the end the second group adds its sums into the first's through LDS (in that
// order, so the result is the two halves' sums added once, as a 2-way k split would add them) and
// the first stores.  For calls whose weight rows give too few workgroups for the chip and are not
// split: each wave then walks half the stages, and two waves share each SIMD, with no partial
// sums in memory and no second launch.
// PAIR: a SwiGLU pair (Q8Group swiglu), a form of its own so the other calls carry none of it.
template <int MT, int S, int NW, bool XS, int KS = 1, bool PAIR = false>
__global__ __launch_bounds__(64 * NW * KS) __attribute__((amdgpu_waves_per_eu(2)))
void linear_q8p_stream_kernel(Q8Args a, Q8Group grp, const _Float16 *xcvt) {
    static_assert(KS == 1 || KS == 2, "one or two stage groups");
    constexpr int NB = kQ8StageBlocks;
    constexpr int NT = 64 * NW;                   // threads of one stage group
    constexpr int SLABS = NW * S;                 // slabs of 32 weight rows per workgroup (NW waves)
    constexpr int PIECES = NB * MT * 4;           // 1 KB pieces of an x stage
    constexpr int XL = PIECES / NW;               // pieces each wave copies (XS = false)
    static_assert(PIECES % NW == 0, "every wave copies whole pieces of the x stage");
    constexpr int STAGE_HALVES = PIECES * 512;
    constexpr int XQ = XS ? MT * 32 * kQ8StageK / 4 / NT : 1; // 16-byte x loads per thread (XS = true)
    static_assert(!XS || XQ * 4 * NT == MT * 32 * kQ8StageK, "every thread loads whole quads of the x stage");
    __shared__ __align__(16) _Float16 xs_all[KS][2][STAGE_HALVES];

    const int lane = threadIdx.x & 63;
    const int wave_all = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); // uniform: the LDS DMA base is per wave
    const int kg = KS == 1 ? 0 : wave_all / NW;                    // stage group
    const int wave = KS == 1 ? wave_all : wave_all - kg * NW;      // wave within the group: its slabs
    // this wave's weight set and its workgroup's index within the set.  A SwiGLU pair: the first
    // NW / 2 waves take the gate's slabs and the others the up's slabs over the same columns.
    constexpr bool pair = PAIR;
    constexpr int HW = NW / 2;
    const int set = pair ? (wave >= HW ? 1 : 0) : q8_group_of_block(grp, (int)blockIdx.x);
    const int bx = (int)blockIdx.x - (pair ? 0 : q8_pick(grp.block_start, set));
    const Q8Packed w = {q8_pick(grp.q, set), q8_pick(grp.scales, set), q8_pick(grp.n_slabs, set), grp.n_chunks};
    a.n = q8_pick(grp.n, set);
    a.bias = q8_pick(grp.bias, set);
    a.out = q8_pick(grp.out, set);
    a.part = q8_pick(grp.part, set);
    // a call of more rows than one x stage holds runs gridDim.z blocks of 32 MT rows (XS only):
    // block z takes rows r0 = 32 MT z .. of x and of the outputs; the partial sums keep the whole
    // call's [split][m][n] layout
    const int m_all = a.m;
    const int r0 = (int)blockIdx.z * MT * 32;
    a.m = min(MT * 32, m_all - r0);
    a.x += (int64_t)r0 * a.k;

    const int tid = KS == 1 ? (int)threadIdx.x : (int)threadIdx.x - kg * NT; // thread within the group
    _Float16(&xs)[2][STAGE_HALVES] = xs_all[kg];
    const int r32 = lane & 31, g = lane >> 5;
    const int hw = pair ? wave - set * HW : wave;   // the wave's place among its set's waves
    const int slab0 = bx * (pair ? HW * S : SLABS) + hw * S; // this wave's first slab
    const int split = blockIdx.y;
    const int n_stages = (a.k + NB * kQ8Block - 1) / (NB * kQ8Block);
    const int w_begin = split * a.chunks_per_split * 2;
    const int w_end = min(w_begin + a.chunks_per_split * 2, n_stages);
    // this group's stages (whole 2-stage turns for the first group, so both groups run as many
    // turns and meet the same barriers)
    const int half = KS == 1 ? w_end - w_begin : ((w_end - w_begin + 3) / 4) * 2;
    const int t_begin = min(w_begin + kg * half, w_end);
    const int t_end = KS == 1 ? w_end : min(t_begin + half, w_end);
    const int turns = (half + 1) / 2; // 2-stage loop turns, the same in every group

    // XS: x [m][k] f32, rows past m read as 0 (range), columns past k get an out-of-range offset;
    // otherwise the call's split x chunks
    const __amdgpu_buffer_rsrc_t x_src =
        XS ? rsrc(a.x, (uint32_t)a.m * (uint32_t)a.k * 4u) : rsrc(xcvt, (uint32_t)w.n_chunks * 2u * (uint32_t)PIECES * 1024u);
    // slabs past the matrix (the last workgroup's) read as 0
    const int live = __builtin_amdgcn_readfirstlane(max(0, min(S, w.n_slabs - slab0)));
    const int64_t slab_q = (int64_t)w.n_chunks * kQ8ChunkBlocks * 1024;
    const int64_t slab_s = (int64_t)w.n_chunks * 32 * kQ8ChunkBlocks * 4;
    const __amdgpu_buffer_rsrc_t q_src = rsrc(w.q + (int64_t)slab0 * slab_q, (uint32_t)(live * slab_q));
    const __amdgpu_buffer_rsrc_t s_src =
        rsrc(reinterpret_cast<const char *>(w.scales) + (int64_t)slab0 * slab_s, (uint32_t)(live * slab_s));

    // XS: x quad e of this thread in a stage is row x_r0 + XR e, k 4 (tid % 32) of the stage; 32
    // consecutive threads read 512 contiguous bytes of a row.  The per-lane part of the offset is
    // one VGPR; the row step and the stage's k go in the scalar offset.  The quad's place in the
    // A-operand order: block, k-step and half of a lane's 8 elements follow the column, the m-tile
    // and lane the row.
    constexpr int XR = NT / 32; // rows between a thread's quads
    const int x_r0 = tid >> 5, x_c = 4 * (tid & 31);
    const uint32_t x_lane = ((uint32_t)x_r0 * (uint32_t)a.k + (uint32_t)x_c) * 4u;
    const uint32_t x_rstep = (uint32_t)XR * (uint32_t)a.k * 4u;
    const int x_b = x_c >> 5, x_kb = x_c & 31;
    const int x_s = (x_kb >> 3) & 1, x_j = x_kb & 7;

    // stage t: its x (into LDS buffer `buf`, or into xr), then this wave's weights and scales into
    // (wq, sc).  Past the last stage (t >= t_end) the same loads go out with out-of-range offsets:
    // they return zeros without touching memory, and every path through the loop then has the same
    // loads in flight, so the compiler's in-order wait counts stay exact.
    auto issue = [&](int t, int buf, f32x4 (&xr)[XQ], u32x4 (&wq)[S][NB], f32x4 (&sc)[S]) {
        const bool live_t = t < t_end;
        if constexpr (XS) {
            const uint32_t xv = live_t && t * kQ8StageK + x_c < a.k ? x_lane : kOutOfRange;
#pragma unroll
            for (int e = 0; e < XQ; ++e)
                xr[e] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               x_src, (int)xv, (int)((uint32_t)e * x_rstep + (uint32_t)(t * kQ8StageK) * 4u), 0));
        } else {
#pragma unroll
            for (int u = 0; u < XL; ++u) {
                const int piece = wave + NW * u;
                const uint32_t off = live_t ? (uint32_t)((t * PIECES + piece) * 1024 + lane * 16) : kOutOfRange;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    x_src, (__attribute__((address_space(3))) void *)(&xs[buf][piece * 512]), 16, off, 0, 0, 0);
            }
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint32_t off = live_t ? (uint32_t)(s * slab_q + ((int64_t)(t * NB + b) * 64 + lane) * 16)
                                            : kOutOfRange;
                wq[s][b] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(q_src, (int)off, 0, kQ8CachePolicyNT));
            }
            // scales of blocks 4 (t % 2) .. +4 of chunk t / 2, this lane's row
            const uint32_t off =
                live_t ? (uint32_t)(s * slab_s + (((t >> 1) * 32 + r32) * kQ8ChunkBlocks + 4 * (t & 1)) * 4)
                       : kOutOfRange;
            sc[s] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(s_src, (int)off, 0, kQ8CachePolicyNT));
        }
    };
    // XS: the stage's x quads, split into f16 hi/lo halves, into LDS buffer `buf` (a quad is half of
    // one lane's 8-element piece)
    auto put_x = [&](int buf, const f32x4 (&xr)[XQ]) {
        if constexpr (XS) {
#pragma unroll
            for (int e = 0; e < XQ; ++e) {
                const int row = x_r0 + XR * e;
                const int i = row >> 5, l = (row & 31) + 32 * (x_kb >> 4);
                half4 hi, lo;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    hi[c] = (_Float16)xr[e][c];
                    lo[c] = (_Float16)(xr[e][c] - (float)hi[c]);
                }
                *reinterpret_cast<half4 *>(&xs[buf][q8_xs_at<MT>(x_b, i, 0, x_s, l) + x_j]) = hi;
                *reinterpret_cast<half4 *>(&xs[buf][q8_xs_at<MT>(x_b, i, 1, x_s, l) + x_j]) = lo;
            }
        }
    };

    f32x16 acc[MT][S];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int s = 0; s < S; ++s) acc[i][s] = (f32x16){0};

    auto compute = [&](int buf, const u32x4 (&wq)[S][NB], const f32x4 (&sc)[S]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            half8 ah[MT][2], al[MT][2];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    ah[i][s] = *reinterpret_cast<const half8 *>(&xs[buf][q8_xs_at<MT>(b, i, 0, s, lane)]);
                    al[i][s] = *reinterpret_cast<const half8 *>(&xs[buf][q8_xs_at<MT>(b, i, 1, s, lane)]);
                }
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const half8 w0 = int8x8_to_half8(wq[s][b][0], wq[s][b][1]);
                const half8 w1 = int8x8_to_half8(wq[s][b][2], wq[s][b][3]);
                const float scb = sc[s][b];
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    f32x16 tt = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], w0, (f32x16){0}, 0, 0, 0);
                    tt = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], w0, tt, 0, 0, 0);
                    tt = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], w1, tt, 0, 0, 0);
                    tt = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], w1, tt, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][s][r] = __builtin_fmaf(tt[r], scb, acc[i][s][r]);
                }
            }
        }
    };

    // Two weight and scale register sets (A for even stages, B for odd) so every index is static;
    // with XS one x register set, written into LDS at the top of its stage and then reloaded.
    f32x4 xr[XQ];
    u32x4 wqA[S][NB], wqB[S][NB];
    f32x4 scA[S], scB[S];
    constexpr int LOADS = S * (NB + 1); // weight and scale loads of one stage, issued after its x
    issue(t_begin, 0, xr, wqA, scA);
    for (int turn = 0, t = t_begin; KS == 1 ? t < t_end : turn < turns; ++turn, t += 2) {
        // stage t (set A, buffer 0)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(q8_vmcnt(LOADS));
        put_x(0, xr);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        issue(t + 1, 1, xr, wqB, scB);
        __builtin_amdgcn_sched_barrier(0);
        if (KS == 1 || t < t_end) compute(0, wqA, scA); // the second group's may be empty
        // stage t + 1 (set B, buffer 1); a no-op past the end (its loads returned zeros)
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(q8_vmcnt(LOADS));
        put_x(1, xr);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        issue(t + 2, 0, xr, wqA, scA);
        __builtin_amdgcn_sched_barrier(0);
        if (t + 1 < t_end) compute(1, wqB, scB);
    }
    __builtin_amdgcn_s_waitcnt(q8_vmcnt(0)); // the last, out-of-range prefetch
    if constexpr (KS == 2) {
        // the second group's sums into the first's, through the (now free) x buffers: lane-major
        // per (wave, m-tile, slab, register), conflict-free
        float *red = reinterpret_cast<float *>(&xs_all[0][0][0]);
        static_assert(NW * MT * S * 16 * 64 * 4 <= (int)sizeof(xs_all), "the sums fit in the x buffers");
        __syncthreads(); // every wave is past its last compute
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int s = 0; s < S; ++s)
#pragma unroll
                    for (int r = 0; r < 16; ++r) red[(((wave * MT + i) * S + s) * 16 + r) * 64 + lane] = acc[i][s][r];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int s = 0; s < S; ++s)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][s][r] += red[(((wave * MT + i) * S + s) * 16 + r) * 64 + lane];
        }
        // an unsplit SwiGLU pair's second group stays for the barriers below
        if (kg == 1 && !(PAIR && a.n_split == 1)) return;
    }

    // an unsplit SwiGLU pair: the up waves hand their values (with bias, as the call would store
    // them) to the gate waves through the freed x buffers (past the two groups' exchange), which
    // store silu(gate) * up
    constexpr int RED2 = KS == 2 ? NW * MT * S * 16 * 64 : 0;
    float *red = reinterpret_cast<float *>(&xs_all[0][0][0]) + RED2;
    static_assert((RED2 + HW * MT * S * 16 * 64) * 4 <= (int)sizeof(xs_all), "the up values fit in the x buffers");
    if (PAIR && a.n_split == 1) {
        __syncthreads(); // every wave is past its last compute (and the first group's sums are whole)
        if (kg == 0 && set == 1) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int col = (slab0 + s) * 32 + r32;
                const float bj = (a.bias && col < a.n) ? a.bias[col] : 0.f;
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) red[(((hw * MT + i) * S + s) * 16 + r) * 64 + lane] = acc[i][s][r] + bj;
            }
        }
        __syncthreads();
        if (kg == 1 || set == 1) return;
    }
    float *dst = (a.n_split > 1 ? a.part + (int64_t)split * m_all * a.n : a.out) + (int64_t)r0 * a.n;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int col = (slab0 + s) * 32 + r32;
        if (col >= a.n) continue;
        const float bj = (a.n_split == 1 && a.bias) ? a.bias[col] : 0.f;
        if (PAIR && a.n_split == 1) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (row < a.m)
                        dst[(int64_t)row * a.n + col] =
                            zwg_ew::silu_mul(acc[i][s][r] + bj, red[(((hw * MT + i) * S + s) * 16 + r) * 64 + lane]);
                }
            continue;
        }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (row < a.m) {
                    if (a.n_split > 1) dst[(int64_t)row * a.n + col] = acc[i][s][r];
                    else zwg_ew::epilogue_store(&dst[(int64_t)row * a.n + col], acc[i][s][r] + bj, a.epi);
                }
            }
    }
}

// out[i][o] (row stride ldo) = epilogue(sum over splits (in split order) of part[split][i][o],
// + bias[o]).  V consecutive elements of one row per thread (V = 4 needs n % 4 == 0 and 16-byte
// aligned partials).  The loads of up to kSumBatch splits are all issued before the first add, so
// a sum waits for one memory latency per batch rather than one per split; the adds stay in split
// order.
constexpr int kSumBatch = 16;
template <int V>
__global__ __launch_bounds__(256) void linear_split_sum_kernel(const float *part, const float *bias, float *out,
                                                              int64_t mn, int32_t n, int32_t n_split, uint32_t epi,
                                                              int64_t ldo) {
    using vec = typename std::conditional<V == 1, float, float __attribute__((ext_vector_type(4)))>::type;
    static_assert(V == 1 || V == 4, "one or four elements per thread");
    const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
    if (e >= mn) return;
    const vec *p = reinterpret_cast<const vec *>(part + e);
    const int64_t step = mn / V;
    vec s{};
    for (int q0 = 0; q0 < n_split; q0 += kSumBatch) {
        vec v[kSumBatch];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j)
            if (q0 + j < n_split) v[j] = p[(q0 + j) * step];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j)
            if (q0 + j < n_split) s = q0 + j == 0 ? v[j] : s + v[j];
    }
    const int64_t row = e / n, col = e - row * n;
    if constexpr (V == 1) {
        zwg_ew::epilogue_store(&out[row * ldo + col], bias ? s + bias[col] : s, epi);
    } else {
#pragma unroll
        for (int v = 0; v < V; ++v)
            zwg_ew::epilogue_store(&out[row * ldo + col + v], bias ? s[v] + bias[col + v] : s[v], epi);
    }
}

// The split sum over a group: element e of the concatenated outputs is element e - elem_start[j]
// of set j, summed over the splits in split order, + bias, through the epilogue.
__global__ __launch_bounds__(256) void linear_split_sum_group_kernel(Q8Group grp, int32_t m, int32_t n_split,
                                                                    uint32_t epi) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= grp.elem_start[kQ8MaxGroup]) return;
    const int set = q8_group_of_elem(grp, e);
    const int64_t le = e - q8_pick(grp.elem_start, set);
    const int32_t n = q8_pick(grp.n, set);
    const int64_t mn = (int64_t)m * n;
    const float *part = q8_pick(grp.part, set);
    const float *bias = q8_pick(grp.bias, set);
    const float *p = part + le;
    float s = 0.f;
    for (int q0 = 0; q0 < n_split; q0 += kSumBatch) { // loads of a batch issued together, adds in split order
        float v[kSumBatch];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j)
            if (q0 + j < n_split) v[j] = p[(q0 + j) * mn];
#pragma unroll
        for (int j = 0; j < kSumBatch; ++j)
            if (q0 + j < n_split) s = q0 + j == 0 ? v[j] : s + v[j];
    }
    if (bias) s += bias[le % n];
    zwg_ew::epilogue_store(&q8_pick(grp.out, set)[le], s, epi);
}

// A split SwiGLU pair's sum (Q8Group swiglu): out[0][e] = silu(gate) * up, gate and up each their
// splits added in split order then their bias, as linear_split_sum_group_kernel forms them, then
// zwg_ew::silu_mul (the separate SiLU-mul kernel's function).  e over m n[0].
__global__ __launch_bounds__(256) void linear_split_sum_swiglu_kernel(Q8Group grp, int32_t m, int32_t n_split) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int32_t n = grp.n[0];
    const int64_t mn = (int64_t)m * n;
    if (e >= mn) return;
    float gu[2];
#pragma unroll
    for (int set = 0; set < 2; ++set) {
        const float *p = (set ? grp.part[1] : grp.part[0]) + e;
        float s = 0.f;
        for (int q0 = 0; q0 < n_split; q0 += kSumBatch) {
            float v[kSumBatch];
#pragma unroll
            for (int j = 0; j < kSumBatch; ++j)
                if (q0 + j < n_split) v[j] = p[(q0 + j) * mn];
#pragma unroll
            for (int j = 0; j < kSumBatch; ++j)
                if (q0 + j < n_split) s = q0 + j == 0 ? v[j] : s + v[j];
        }
        const float *bias = set ? grp.bias[1] : grp.bias[0];
        if (bias) s += bias[e % n];
        gu[set] = s;
    }
    grp.out[0][e] = zwg_ew::silu_mul(gu[0], gu[1]);
}

// The q/k/v group's split sum with the cache append fused into its stores (set 0 q, 1 k, 2 v of a
// Q8Group; n = heads * D).  Where the split sum writes rows and kv_append_kernel then reads them
// back, this kernel takes the same sums -- the splits added in split order, then the bias -- and
// does what the append does with them:
//   - q and k at their token's position get NeoX rotary positions (pairs (j, j + D/2), rounded
//     product by product as the reference does, src/llm.zig:221-238) when the cache has tables;
//   - q is written to q_out; k into the key cache, transposed ([head][dim][n_ctx]) or as a row; v
//     as a row; a token whose position is outside [0, n_ctx) writes no cache rows and an unrotated q.
// So the caches and q equal, bit for bit, the group call into rows followed by zwg_kv_append_batch.
// A thread takes one (token, set, head, 4 dims j .. j+3) and the 4 dims j + D/2 .. of the pair.
struct Q8KvStore {
    float *q_out;           // [m][n_head * D]
    float *k_cache;         // the layer's caches: token i's sequence seq0 + i at + (seq0 + i) * per_seq
    float *v_cache;
    const float *cos;       // [n_ctx][D/2], or nullptr: no rotary positions
    const float *sin;
    const int32_t *pos_dev; // [m] positions, or nullptr: token i at pos0 + i
    int32_t *n_kv_out;      // or nullptr: [m] keys each sequence's cache then holds, pos + 1 (0 off the cache)
    int64_t per_seq;
    int32_t seq0, n_ctx, n_head, n_head_kv, kt;
    int32_t pos0;     // the first position when pos_dev is nullptr
    int32_t seq_step; // token i's sequence is seq0 + i seq_step: 1 (a decode step), 0 (one sequence's rows)
    int32_t d; // the kernel's D (host side: which instantiation)
};

template <int D>
__global__ __launch_bounds__(256) void linear_split_sum_qkv_kernel(Q8Group grp, Q8KvStore kv, int32_t m,
                                                                  int32_t n_split) {
#pragma clang fp contract(off) // the rotation rounds each product and sum, as the reference does
    constexpr int HALF = D / 2, QH = D / 8; // pair quads per head
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_tok = (kv.n_head + 2 * kv.n_head_kv) * QH;
    if (e >= (int64_t)m * per_tok) return;
    const int i = (int)(e / per_tok);
    int u = (int)(e - (int64_t)i * per_tok);
    const int set = u < kv.n_head * QH ? 0 : u < (kv.n_head + kv.n_head_kv) * QH ? 1 : 2;
    u -= set == 0 ? 0 : set == 1 ? kv.n_head * QH : (kv.n_head + kv.n_head_kv) * QH;
    const int h = u / QH, j = 4 * (u - h * QH);
    const int32_t n = q8_pick(grp.n, set);
    const int64_t mn = (int64_t)m * n;
    const float *part = q8_pick(grp.part, set) + (int64_t)i * n + h * D + j;
    const float *bias = q8_pick(grp.bias, set);
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
    for (int q0 = 0; q0 < n_split; q0 += kSumBatch) { // as linear_split_sum_group_kernel: loads first
        f4 vl[kSumBatch], vh[kSumBatch];
#pragma unroll
        for (int t = 0; t < kSumBatch; ++t)
            if (q0 + t < n_split) {
                vl[t] = *reinterpret_cast<const f4 *>(part + (q0 + t) * mn);
                vh[t] = *reinterpret_cast<const f4 *>(part + (q0 + t) * mn + HALF);
            }
#pragma unroll
        for (int t = 0; t < kSumBatch; ++t)
            if (q0 + t < n_split) {
                lo = q0 + t == 0 ? vl[t] : lo + vl[t];
                hi = q0 + t == 0 ? vh[t] : hi + vh[t];
            }
    }
    if (bias) {
        const f4 bl = *reinterpret_cast<const f4 *>(bias + h * D + j);
        const f4 bh = *reinterpret_cast<const f4 *>(bias + h * D + j + HALF);
        lo += bl;
        hi += bh;
    }
    const int p = kv.pos_dev ? kv.pos_dev[i] : kv.pos0 + i;
    const bool live = p >= 0 && p < kv.n_ctx;
    if (kv.n_kv_out && set == 0 && h == 0 && j == 0) kv.n_kv_out[i] = live ? p + 1 : 0;
    if (set < 2 && kv.cos && live) {
        const f4 c = *reinterpret_cast<const f4 *>(kv.cos + (int64_t)p * HALF + j);
        const f4 s = *reinterpret_cast<const f4 *>(kv.sin + (int64_t)p * HALF + j);
        const f4 x0 = lo, x1 = hi;
        lo = x0 * c - x1 * s;
        hi = x0 * s + x1 * c;
    }
    if (set == 0) {
        float *qr = kv.q_out + (int64_t)i * kv.n_head * D + h * D + j;
        *reinterpret_cast<f4 *>(qr) = lo;
        *reinterpret_cast<f4 *>(qr + HALF) = hi;
        return;
    }
    if (!live) return;
    const int kvw = kv.n_head_kv * D;
    const int64_t seq = (int64_t)(kv.seq0 + i * kv.seq_step) * kv.per_seq;
    if (set == 1 && kv.kt) {
        float *kc = kv.k_cache + seq + (int64_t)(h * D + j) * kv.n_ctx + p;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            kc[(int64_t)t * kv.n_ctx] = lo[t];
            kc[(int64_t)(t + HALF) * kv.n_ctx] = hi[t];
        }
        return;
    }
    float *row = (set == 1 ? kv.k_cache : kv.v_cache) + seq + (int64_t)p * kvw + h * D + j;
    *reinterpret_cast<f4 *>(row) = lo;
    *reinterpret_cast<f4 *>(row + HALF) = hi;
}

// A one-set call's split sum added to the residual stream and normalised, for the decoder blocks'
// ops.linear + ops.add + next ops.layerNorm (src/decoder.zig:185-188, :192-195, :200 with the
// next block's :178) and Qwen2's + ops.rmsNorm (src/llm.zig:203-204, :206-207 with :178): row i
// of x += sum over splits (in split order) of part[s][i] + bias -- as
// linear_split_sum_group_kernel with the add epilogue forms it -- then ln_out[i] = the norm of
// x[i] (NORM: zwg_ew::kNormLayer or kNormRms, through the functions layer_norm_kernel and
// rms_norm_kernel use).  So x and ln_out equal the split sum and the norm launch bit for bit.  One wave per row of n <= 256 R floats; the
// residual row, the bias and the partials of B splits at a time are loaded before any add.  One
// one-wave workgroup per row.
struct Q8ResLn {
    float *x; // [m][n] residual stream, updated in place
    const float *ln_w, *ln_b; // ln_b unused by the RMS norm
    float *ln_out; // [m][n]
    float eps;
    int32_t norm; // zwg_ew::kNormLayer or kNormRms (host side: which instantiation)
    // nullptr, or the normalised rows also split into f16 hi/lo halves for the next 64-row call
    // (linear_q8_xprep_kernel's layout and values, rows m .. 63 zero); the one-thread-per-column
    // kernel only
    _Float16 *xcvt;
};

template <int R, int NORM>
__global__ __launch_bounds__(64) void linear_split_sum_add_ln_kernel(const float *part, const float *bias, Q8ResLn r,
                                                                     int32_t m, int32_t n, int32_t n_split) {
#pragma clang fp contract(off)
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int B = 48 / R < 16 ? 48 / R : 16; // splits whose loads go out together (B R float4 per lane)
    const int lane = threadIdx.x;
    const int row = (int)blockIdx.x; // one wave per workgroup, one row per wave
    if (row >= m) return;
    const int n4 = n >> 2;
    const int64_t step = (int64_t)m * n4; // float4s of one split
    const f4 *p = reinterpret_cast<const f4 *>(part) + (int64_t)row * n4;
    // the residual row and the bias first: their loads share the partials' round trip
    f4 *xr = reinterpret_cast<f4 *>(r.x + (int64_t)row * n);
    f4 xo[R], bo[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        if (c < n4) {
            xo[i] = xr[c];
            bo[i] = bias ? reinterpret_cast<const f4 *>(bias)[c] : (f4){0.f, 0.f, 0.f, 0.f};
        }
    }
    f4 s[R];
#pragma unroll
    for (int i = 0; i < R; ++i) s[i] = (f4){0.f, 0.f, 0.f, 0.f};
    for (int q0 = 0; q0 < n_split; q0 += B) {
        f4 t[B][R];
#pragma unroll
        for (int j = 0; j < B; ++j)
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int c = lane + 64 * i;
                if (q0 + j < n_split && c < n4) t[j][i] = p[(q0 + j) * step + c];
            }
#pragma unroll
        for (int j = 0; j < B; ++j)
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int c = lane + 64 * i;
                if (q0 + j < n_split && c < n4) s[i] = q0 + j == 0 ? t[j][i] : s[i] + t[j][i];
            }
    }
    zwg_ew::ew_f32x4 v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        if (c < n4) {
            f4 val = s[i];
            if (bias) val = val + bo[i];
            const f4 nx = xo[i] + val;
            xr[c] = nx;
            v[i] = nx;
        } else {
            v[i] = (zwg_ew::ew_f32x4){0.f, 0.f, 0.f, 0.f};
        }
    }
    zwg_ew::norm_regs<NORM, R>(v, lane, n4, r.ln_w, r.ln_b, r.eps, r.ln_out + (int64_t)row * n);
}

// The same sums, residual add and norm with one thread per float4 column (R waves per row, n <=
// 256 R floats): each thread has up to 24 of its column's splits in flight at once, where the
// one-wave kernel walks R columns per lane in batches of 48 / R splits (the Qwen2.5-1.5B down
// projection's 35 splits of 1536-float rows: 18 batches of loads one after another per wave).
// The new row goes through LDS to the first wave, which normalises it with norm_regs exactly as
// the one-wave kernel does (so the two give the same bits).
template <int R, int NORM>
__global__ __launch_bounds__(64 * R) void linear_split_sum_add_ln_wide_kernel(const float *part, const float *bias,
                                                                              Q8ResLn r, int32_t m, int32_t n,
                                                                              int32_t n_split) {
#pragma clang fp contract(off)
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int B = 24;
    __shared__ f4 rowbuf[64 * R];
    const int c = threadIdx.x; // this thread's float4 column
    const int row = (int)blockIdx.x;
    if (row >= m) return;
    const int n4 = n >> 2;
    const bool live = c < n4;
    const int64_t step = (int64_t)m * n4;
    const f4 *p = reinterpret_cast<const f4 *>(part) + (int64_t)row * n4 + c;
    f4 *xr = reinterpret_cast<f4 *>(r.x + (int64_t)row * n);
    f4 xo = {0.f, 0.f, 0.f, 0.f}, bo = {0.f, 0.f, 0.f, 0.f};
    if (live) {
        xo = xr[c];
        if (bias) bo = reinterpret_cast<const f4 *>(bias)[c];
    }
    f4 s = {0.f, 0.f, 0.f, 0.f};
    for (int q0 = 0; q0 < n_split; q0 += B) {
        f4 t[B];
#pragma unroll
        for (int j = 0; j < B; ++j)
            if (live && q0 + j < n_split) t[j] = p[(q0 + j) * step];
#pragma unroll
        for (int j = 0; j < B; ++j)
            if (live && q0 + j < n_split) s = q0 + j == 0 ? t[j] : s + t[j];
    }
    f4 nx = {0.f, 0.f, 0.f, 0.f};
    if (live) {
        f4 val = s;
        if (bias) val = val + bo;
        nx = xo + val;
        xr[c] = nx;
    }
    rowbuf[c] = nx;
    __syncthreads();
    if (c < 64) {
        zwg_ew::ew_f32x4 v[R];
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = rowbuf[c + 64 * i];
        // with xcvt the normalised row also goes back into rowbuf (past n4 it stays zero)
        zwg_ew::norm_regs<NORM, R>(v, c, n4, r.ln_w, r.ln_b, r.eps, r.ln_out + (int64_t)row * n,
                                   r.xcvt ? rowbuf : nullptr);
    }
    if (r.xcvt) {
        __syncthreads();
        const int n_cols = (n + kQ8Chunk - 1) / kQ8Chunk * (kQ8Chunk / 4); // float4 columns of whole chunks
        if (c < n_cols) {
            q8_xs_store<2>(r.xcvt, row, 4 * c, rowbuf[c]);
            for (int z = row + m; z < 64; z += m) q8_xs_store<2>(r.xcvt, z, 4 * c, (f32x4){0.f, 0.f, 0.f, 0.f});
        }
    }
}

// A decode step's token embeddings from the packed int8 token embedding (the tied output
// projection): x[i] = te.row(tok[i]) + pe[pos[i]] -- gemm.Q8.row (src/gemm.zig:257-265, q * scale
// in f32) then ops.add (src/decoder.zig:171-174) -- and ln_out[i] = the norm of x[i] (the first
// block's attn_ln, src/decoder.zig:178; for Qwen2, no position rows and the first block's RMS
// norm, src/llm.zig:175-178).  A token outside
// [0, n_vocab) gives a zero embedding row; a position outside [0, pe_rows) adds no position row
// (pos may be null when there are none).
// One wave per row of n <= 256 R floats; a lane's float4 is 4 bytes of one 16-byte lane piece of
// its block's tile (Q8Packed).
template <int R, int NORM>
__global__ __launch_bounds__(64) void q8p_embed_ln_kernel(Q8Packed te, int32_t n_vocab, const int32_t *tok,
                                                          const float *pe, const int32_t *pos, int32_t pe_rows,
                                                          int32_t m, int32_t n, float *x, Q8ResLn r) {
#pragma clang fp contract(off)
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x;
    const int row = (int)blockIdx.x; // one wave per workgroup, one row per wave
    if (row >= m) return;
    const int n4 = n >> 2;
    const int t = tok[row], ps = pos ? pos[row] : -1;
    const bool t_ok = t >= 0 && t < n_vocab, p_ok = ps >= 0 && ps < pe_rows;
    const int slab = t_ok ? t >> 5 : 0, r32 = t & 31;
    const int nbp = te.n_chunks * kQ8ChunkBlocks;
    zwg_ew::ew_f32x4 v[R];
    f4 *xr = reinterpret_cast<f4 *>(x + (int64_t)row * n);
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int c = lane + 64 * i;
        f4 val = {0.f, 0.f, 0.f, 0.f};
        if (c < n4) {
            if (t_ok) {
                const int k0 = 4 * c, b = k0 >> 5;
                const uint32_t w4 = *reinterpret_cast<const uint32_t *>(
                    te.q + (((int64_t)slab * nbp + b) * 64 + r32 + 32 * ((k0 & 31) >> 4)) * 16 + (k0 & 15));
                const float sc =
                    te.scales[(((int64_t)slab * te.n_chunks + (b >> 3)) * 32 + r32) * kQ8ChunkBlocks + (b & 7)];
#pragma unroll
                for (int e = 0; e < 4; ++e) val[e] = (float)(int8_t)(uint8_t)(w4 >> (8 * e)) * sc;
            }
            if (p_ok) val = val + reinterpret_cast<const f4 *>(pe + (int64_t)ps * n)[c];
            xr[c] = val;
        }
        v[i] = val;
    }
    zwg_ew::norm_regs<NORM, R>(v, lane, n4, r.ln_w, r.ln_b, r.eps, r.ln_out + (int64_t)row * n);
}

} // namespace zwg_lin
