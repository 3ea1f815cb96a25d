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
//   rows and walks k in chunks of 256 (8 blocks).  Each chunk of x ([32*MT][256] f32) is split
//   into hi/lo halves once per workgroup and parked in LDS in the exact order the MFMA A operand
//   wants it, so a wave's operand read is 1 KB contiguous (conflict-free ds_read_b128).
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

#include "linear_kernel.hpp"

namespace zwg_lin {

constexpr int kQ8Block = 32;                // src/gemm.zig:194
constexpr int kQ8Chunk = 256;               // k per LDS chunk of the stream kernel
constexpr int kQ8ChunkBlocks = kQ8Chunk / kQ8Block;
constexpr int kQ8Threads = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Q8Args {
    const float *x;      // [m][k]
    const int8_t *q;     // [n][k]
    const float *scales; // [n][nb]
    const float *bias;   // [n] or nullptr
    float *out;          // [m][n]
    float *part;         // [n_split][m][n] when n_split > 1
    int32_t m, n, k, nb;
    int32_t chunks_per_split, n_split;
};

// Stream kernel LDS layout of one chunk of x: [block][m-tile][hi/lo][k-step][lane][8 halves].
// Lane l, k-step s of (block b, m-tile i) holds x[32 i + l % 32][kb + 16 (l / 32) + 8 s + 0..7].
template <int MT>
__device__ __forceinline__ int q8_xs_at(int b, int i, int hl, int s, int lane) {
    return ((((b * MT + i) * 2 + hl) * 2 + s) * 64 + lane) * 8;
}

template <int MT, int S>
__global__ __launch_bounds__(kQ8Threads) void linear_q8_stream_kernel(Q8Args a) {
    constexpr int NB = kQ8ChunkBlocks;
    constexpr int XL = MT * 32 * kQ8Chunk / 4 / kQ8Threads; // float4 loads of x per thread per chunk
    constexpr int ROWS = 4 * S * 32;                         // weight rows per workgroup
    __shared__ __align__(16) _Float16 xs[MT * NB * 2 * 2 * 64 * 8];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int n0 = blockIdx.x * ROWS;
    const int wrow0 = wave * S * 32; // this wave's first row within the workgroup's slab group
    const int split = blockIdx.y;
    const int n_chunks = (a.k + kQ8Chunk - 1) / kQ8Chunk;
    const int c_begin = split * a.chunks_per_split;
    const int c_end = min(c_begin + a.chunks_per_split, n_chunks);

    // x: rows past m read as 0 (range ends at row m); q / scales: rows past n read as 0.
    const __amdgpu_buffer_rsrc_t x_src = rsrc(a.x, (uint32_t)((int64_t)a.m * a.k * 4));
    const int rows_w = min(ROWS, a.n - n0);
    const __amdgpu_buffer_rsrc_t q_src = rsrc(a.q + (int64_t)n0 * a.k, (uint32_t)((int64_t)rows_w * a.k));
    const __amdgpu_buffer_rsrc_t s_src = rsrc(a.scales + (int64_t)n0 * a.nb, (uint32_t)((int64_t)rows_w * a.nb * 4));

    f32x16 acc[MT][S];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int s = 0; s < S; ++s) acc[i][s] = (f32x16){0};

    for (int c = c_begin; c < c_end; ++c) {
        const int k0 = c * kQ8Chunk;
        // x chunk: float4 f covers row f / 64, k = k0 + 4 (f % 64)
        f32x4 xr[XL];
#pragma unroll
        for (int u = 0; u < XL; ++u) {
            const int f = tid + kQ8Threads * u;
            const int row = f / (kQ8Chunk / 4), gk = k0 + 4 * (f % (kQ8Chunk / 4));
            const uint32_t off = gk < a.k ? (uint32_t)(row * a.k + gk) * 4u : kOutOfRange;
            xr[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(x_src, (int)off, 0, 0));
        }
        __syncthreads(); // the previous chunk's operand reads are done
#pragma unroll
        for (int u = 0; u < XL; ++u) {
            const int f = tid + kQ8Threads * u;
            const int row = f / (kQ8Chunk / 4), kk = 4 * (f % (kQ8Chunk / 4));
            const int b = kk >> 5, kb = kk & 31;
            const int gg = kb >> 4, s = (kb >> 3) & 1, j = kb & 7;
            const int i = row >> 5, l = (row & 31) + 32 * gg;
            half4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                hi[e] = (_Float16)xr[u][e];
                lo[e] = (_Float16)(xr[u][e] - (float)hi[e]);
            }
            *reinterpret_cast<half4 *>(&xs[q8_xs_at<MT>(b, i, 0, s, l) + j]) = hi;
            *reinterpret_cast<half4 *>(&xs[q8_xs_at<MT>(b, i, 1, s, l) + j]) = lo;
        }
        __syncthreads();

        // this wave's weights for the chunk: slab s, block b -> 16 bytes per lane, and its scale
        u32x4 wq[S][NB];
        float sc[S][NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int kb = k0 + b * kQ8Block;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int row = wrow0 + s * 32 + r32;
                const uint32_t qoff = kb < a.k ? (uint32_t)(row * a.k + kb + 16 * g) : kOutOfRange;
                const uint32_t soff = kb < a.k ? (uint32_t)(row * a.nb + kb / kQ8Block) * 4u : kOutOfRange;
                wq[s][b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(q_src, (int)qoff, 0, 0));
                sc[s][b] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s_src, (int)soff, 0, 0));
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (k0 + b * kQ8Block >= a.k) break; // uniform: the last chunk may be short
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
                if (row < a.m) dst[(int64_t)row * a.n + col] = acc[i][s][r] + bj;
            }
    }
}

// out[i][o] = sum over splits (in split order) of part[split][i][o], + bias[o].
__global__ __launch_bounds__(256) void linear_split_sum_kernel(const float *part, const float *bias, float *out,
                                                              int64_t mn, int32_t n, int32_t n_split) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= mn) return;
    float s = part[e];
    for (int p = 1; p < n_split; ++p) s += part[(int64_t)p * mn + e];
    if (bias) s += bias[e % n];
    out[e] = s;
}

} // namespace zwg_lin
