// The linear-layer kernel on gfx950 MFMA: out[i][o] = sum_p x[i][p] * w[o][p] (+ b[o]), x f32,
// w f16 or int8 blocks, out f32 (ops.linear with f16 weights, src/ops.zig:283-306,
// src/gemm.zig:117-137; with gemm.Q8 weights, src/gemm.zig:188-351).
//
// Precision.  An f16 weight is exact in f16, and each f32 activation is split into two f16
// terms, x = hi + lo with hi = f16(x) and lo = f16(x - hi): they keep 22 of x's 24 significand
// bits (residual below 2^-21 |x|; a subnormal lo term loses less than 2^-25 absolute).  Both
// products accumulate in f32 on v_mfma_f32_32x32x16_f16, so a dot product carries f32-level
// error, as the reference's f32 FMA chain does, at the f16 MFMA rate.  |x| must stay within
// f16's range (65504); a larger input turns into inf in its output row rather than a wrong
// finite value.
//
// Tiles.  A workgroup of 4 waves computes a BM x BN block of out as 2 x 2 waves, each a
// (BM/2) x (BN/2) block of 32 x 32 MFMA tiles.  K goes through LDS 32 at a time, double-
// buffered, with the next stage's global loads in flight during the current stage's MFMAs:
// x is converted to its hi and lo halves on the way in (each element once per workgroup), w is
// copied as is.  An LDS row is 32 halves (64 bytes, four 16-byte chunks) with chunk c of row r
// stored at c ^ ((r ^ (r >> 2)) & 3): the 16-byte operand reads of a wave (32 rows, two
// chunks) then run at the full LDS read rate on gfx950 (measured: this XOR reads as fast as a
// contiguous block, while (r >> 1) & 3 or an unswizzled 64-byte row reads 1.7-3x slower), with
// no padding, so two workgroups of the 128 x 256 tile fit a CU's LDS.  MFMA operand layout
// (measured on the device): lane l, half s of A is A[l % 32][8 (l / 32) + s], of B is
// B[8 (l / 32) + s][l % 32]; result register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
//
// Int8 block weights (Q8 = true; gemm.Q8, src/gemm.zig:188-351).  A stage of BK = 32 is exactly
// one Q8 block, so the weight tile is widened from int8 to f16 (exact) on its way into LDS, the
// stage's MFMAs accumulate into a zeroed block sum, and the block sum is scaled by the weight
// row's f32 scale into the accumulator (one scale per lane and 32-column tile: the result column
// is the weight row).  The scales of the next stage are loaded with its tiles.
//
// Bounds.  Loads go through buffer descriptors whose range ends at the workgroup's last row of
// x (or w): rows past m (or n) read as 0 in hardware, and a K column past k gets an offset
// beyond the range, so the loop body has no branches.  The host guarantees k % 8 == 0 and a
// per-workgroup range below 2^31 bytes.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "elementwise.hpp"
#include "kv_image.hpp"

namespace zwg_lin {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;                 // K per LDS stage: one 64-byte LDS row
constexpr uint32_t kOutOfRange = 0x80000000u; // a buffer offset past every range the host allows

// Weight formats of the tiled kernel.
constexpr int kWF16 = 0;   // f16 [n][ldw]
constexpr int kWQ8 = 1;    // int8 [n][ldw] + f32 scales [n][nb]
constexpr int kWQ8P = 2;   // int8 + scales packed per slab of 32 rows (linear_q8_kernel.hpp, Q8Packed)

struct LinearArgs {
    const float *x;      // [m][ldx]
    const void *w;       // f16 [n][ldw], int8 [n][ldw], or packed int8 tiles
    const float *scales; // Q8 weights: [n][nb] f32 block scales, or packed scales
    int32_t p_chunks;    // packed weights: chunks of 256 k per slab
    const float *bias;   // [n] or nullptr
    float *out;          // [m][ldo]
    int64_t ldx, ldw, ldo;
    int32_t m, n, k, nb;
    uint32_t epi; // zwg_ew::kEpi*: store v, gelu(v) or out + v, v = x . w + b
    // K split over gridDim.y workgroups when a call has too few tiles to fill the GPU: split s
    // takes k in [s k_split, (s + 1) k_split) (a multiple of BK) and stores its raw sums in
    // part[s][m][n]; a second kernel adds the splits in order, then bias and epilogue
    int32_t k_split;
    float *part;
    // img_kind 1 (K) or 2 (V): the outputs go to `img` as tile images (kv_image.hpp) instead of to
    // out -- rows are (item, key) with img_ctx keys per item (a multiple of 4), columns (head, dim)
    // with img_d dims per head, img_tiles tiles per (item, head); no k split, no epilogue
    _Float16 *img;
    int32_t img_kind, img_ctx, img_d, img_heads, img_tiles;
};

// Eight int8 (two dwords) to eight exact f16: the biased byte b + 128 is placed under the
// exponent bits of 1024.0 (0x64), which gives 1024 + b + 128, and 1152 is taken off in f16.
__device__ __forceinline__ half8 int8x8_to_half8(uint32_t w0, uint32_t w1) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    half8 r;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const uint32_t u = (d ? w1 : w0) ^ 0x80808080u;
        const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
        const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
        r[4 * d + 0] = a[0];
        r[4 * d + 1] = a[1];
        r[4 * d + 2] = b[0];
        r[4 * d + 3] = b[1];
    }
    return r;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// MI355X deals consecutive workgroups round-robin over its 8 XCDs, each with its own L2.  The
// tiles of a call are numbered so that each XCD runs one contiguous range of logical tiles,
// column tiles fastest: the tiles that read the same rows of x run together on one XCD and share
// its L2 instead of each fetching those rows from the fabric.
__device__ __forceinline__ int64_t xcd_logical_tile(int64_t hw, int64_t n) {
    constexpr int X = 8;
    const int64_t xcd = hw % X, local = hw / X, q = n / X, r = n % X;
    return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// half index of (row, 8-half chunk) in a swizzled LDS tile
__device__ __forceinline__ int lds_at(int row, int chunk) { return row * BK + ((chunk ^ ((row ^ (row >> 2)) & 3)) << 3); }

// The kernel's body, taking the arguments by reference (measured 1-2% faster on the base.en
// projections than the same code as the kernel itself, with its by-value argument).
template <int BM, int BN, int WMODE, int NWN, bool KSPLIT>
__device__ __forceinline__ void linear_mfma_body(const LinearArgs &a) {
    // 2 x NWN waves, each a (BM / 2) x (BN / NWN) block of the tile
    constexpr int kThreads = 128 * NWN;
    constexpr bool Q8 = WMODE != kWF16;
    constexpr int WM = BM / 2, WN = BN / NWN; // per wave
    constexpr int TM = WM / 32, TN = WN / 32; // 32 x 32 MFMA tiles per wave
    constexpr int XL = BM * BK / 4 / kThreads; // float4 loads of x per thread per stage
    // 16-byte loads of w per stage: 8 halves (f16) or 16 int8 (Q8) each
    constexpr int W_LOADS = Q8 ? BN * BK / 16 : BN * BK / 8;
    constexpr int WL = (W_LOADS + kThreads - 1) / kThreads;
    static_assert(XL >= 1 && TM >= 1 && TN >= 1, "tile too small for the workgroup");
    static_assert(W_LOADS % 64 == 0, "w loads must cover whole waves");

    __shared__ __align__(16) _Float16 xh[2][BM * BK];
    __shared__ __align__(16) _Float16 xl[2][BM * BK];
    __shared__ __align__(16) _Float16 ws[2][BN * BK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / NWN, wn = wave % NWN;
    const int n_col_tiles = (a.n + BN - 1) / BN;
    const int64_t tile = xcd_logical_tile(blockIdx.x, gridDim.x);
    // KSPLIT: workgroup (tile, s) takes k in [s k_split, (s + 1) k_split); k_lo is 0 otherwise
    const int split = KSPLIT ? (int)blockIdx.y : 0;
    const int k_lo = split * a.k_split;
    const int m0 = (int)(tile / n_col_tiles) * BM, n0 = (int)(tile % n_col_tiles) * BN;
    const int r32 = lane & 31, ch = lane >> 5;

    const int rows_x = min(BM, a.m - m0), rows_w = min(BN, a.n - n0);
    const int wbytes = Q8 ? 1 : 2;
    const __amdgpu_buffer_rsrc_t xr_src = rsrc(a.x + (int64_t)m0 * a.ldx, (uint32_t)(rows_x * a.ldx * 4));
    __amdgpu_buffer_rsrc_t wr_src, sc_src;
    if constexpr (WMODE == kWQ8P) {
        // packed: this tile's slabs n0 / 32 .. ; slabs past the matrix read as 0
        const int64_t slab_q = (int64_t)a.p_chunks * 8 * 1024, slab_s = (int64_t)a.p_chunks * 32 * 8 * 4;
        const int live = (rows_w + 31) / 32;
        wr_src = rsrc(static_cast<const char *>(a.w) + (int64_t)(n0 / 32) * slab_q, (uint32_t)(live * slab_q));
        sc_src = rsrc(reinterpret_cast<const char *>(a.scales) + (int64_t)(n0 / 32) * slab_s, (uint32_t)(live * slab_s));
    } else {
        wr_src = rsrc(static_cast<const char *>(a.w) + (int64_t)n0 * a.ldw * wbytes, (uint32_t)(rows_w * a.ldw * wbytes));
        sc_src = rsrc(Q8 ? a.scales + (int64_t)n0 * a.nb : a.x, Q8 ? (uint32_t)(rows_w * a.nb * 4) : 0u);
    }

    f32x4 xr[XL];
    f32x4 wr[WL]; // raw 16-byte weight loads
    float sc_next[Q8 ? TN : 1];
    // stage loads: x element (row, 4 k) and w element (row, 8 halves or 16 int8 along k)
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int f = tid + kThreads * i;
            const int row = f / (BK / 4), gk = k0 + 4 * (f % (BK / 4));
            const uint32_t off = gk < a.k ? (uint32_t)(row * a.ldx + gk) * 4u : kOutOfRange;
            xr[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr_src, (int)off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            const int f = tid + kThreads * i;
            if (W_LOADS % kThreads != 0 && f >= W_LOADS) break; // whole waves drop out
            uint32_t off;
            if constexpr (WMODE == kWQ8P) {
                // (slab f / 64, lane f % 64) of block k0 / 32: 16 int8 of row 32 slab + lane % 32
                off = (uint32_t)(((f >> 6) * a.p_chunks * 8 + k0 / BK) * 64 + (f & 63)) * 16u;
            } else {
                constexpr int PER_ROW = Q8 ? BK / 16 : BK / 8;
                const int row = f / PER_ROW, gk = k0 + (BK / PER_ROW) * (f % PER_ROW);
                off = gk < a.k ? (uint32_t)(row * a.ldw + gk) * (uint32_t)wbytes : kOutOfRange;
            }
            wr[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wr_src, (int)off, 0, 0));
        }
        if constexpr (Q8) {
            // this lane's weight rows of the next stage: one block scale each (k0 / 32 is the block)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int row = wn * WN + j * 32 + r32;
                uint32_t off;
                if constexpr (WMODE == kWQ8P)
                    off = (uint32_t)((((row >> 5) * a.p_chunks + k0 / 256) * 32 + (row & 31)) * 8 + (k0 / BK) % 8) * 4u;
                else
                    off = k0 < a.k ? (uint32_t)(row * a.nb + k0 / BK) * 4u : kOutOfRange;
                sc_next[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sc_src, (int)off, 0, 0));
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int f = tid + kThreads * i;
            const int row = f / (BK / 4), q = f % (BK / 4);
            half4 hi, lo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hi[j] = (_Float16)xr[i][j];
                lo[j] = (_Float16)(xr[i][j] - (float)hi[j]);
            }
            const int at = lds_at(row, q >> 1) + 4 * (q & 1);
            *reinterpret_cast<half4 *>(&xh[buf][at]) = hi;
            *reinterpret_cast<half4 *>(&xl[buf][at]) = lo;
        }
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            const int f = tid + kThreads * i;
            if (W_LOADS % kThreads != 0 && f >= W_LOADS) break;
            if constexpr (Q8) {
                // 16 int8 of k 16 h .. +16 of one row: two f16 chunks.  Raw: row f / 2, h = f % 2;
                // packed: slab f / 64, lane f % 64 -> row 32 slab + lane % 32, h = lane / 32
                const int row = WMODE == kWQ8P ? ((f >> 6) << 5) + (f & 31) : f >> 1;
                const int c = WMODE == kWQ8P ? 2 * ((f >> 5) & 1) : 2 * (f & 1);
                const uint32_t *u = reinterpret_cast<const uint32_t *>(&wr[i]);
                *reinterpret_cast<half8 *>(&ws[buf][lds_at(row, c)]) = int8x8_to_half8(u[0], u[1]);
                *reinterpret_cast<half8 *>(&ws[buf][lds_at(row, c + 1)]) = int8x8_to_half8(u[2], u[3]);
            } else {
                const int row = f / (BK / 8), c = f % (BK / 8);
                *reinterpret_cast<half8 *>(&ws[buf][lds_at(row, c)]) = __builtin_bit_cast(half8, wr[i]);
            }
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (f32x16){0};

    float sc[Q8 ? TN : 1];
    auto compute = [&](int buf) {
        if constexpr (!Q8) {
#pragma unroll
            for (int kk = 0; kk < BK / 16; ++kk) {
                half8 ah[TM], al[TM], b[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int at = lds_at(wm * WM + i * 32 + r32, 2 * kk + ch);
                    ah[i] = *reinterpret_cast<const half8 *>(&xh[buf][at]);
                    al[i] = *reinterpret_cast<const half8 *>(&xl[buf][at]);
                }
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    b[j] = *reinterpret_cast<const half8 *>(&ws[buf][lds_at(wn * WN + j * 32 + r32, 2 * kk + ch)]);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], acc[i][j], 0, 0, 0);
            }
        } else {
            // the stage is one Q8 block: its sum over 32 k, then scaled into acc
            half8 ah[TM][2], al[TM][2];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int at = lds_at(wm * WM + i * 32 + r32, 2 * kk + ch);
                    ah[i][kk] = *reinterpret_cast<const half8 *>(&xh[buf][at]);
                    al[i][kk] = *reinterpret_cast<const half8 *>(&xl[buf][at]);
                }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                half8 b[2];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    b[kk] = *reinterpret_cast<const half8 *>(&ws[buf][lds_at(wn * WN + j * 32 + r32, 2 * kk + ch)]);
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    f32x16 t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], b[0], (f32x16){0}, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], b[0], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], b[1], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], b[1], t, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(t[r], sc[j], acc[i][j][r]);
                }
            }
        }
    };

    const int n_k = KSPLIT ? min((a.k - k_lo + BK - 1) / BK, a.k_split / BK) : (a.k + BK - 1) / BK;
    load(k_lo);
    store(0);
    if constexpr (Q8) {
#pragma unroll
        for (int j = 0; j < TN; ++j) sc[j] = sc_next[j];
    }
    __syncthreads();
    for (int t = 0; t + 1 < n_k; ++t) {
        load(k_lo + (t + 1) * BK);
        compute(t & 1);
        store((t + 1) & 1);
        if constexpr (Q8) {
#pragma unroll
            for (int j = 0; j < TN; ++j) sc[j] = sc_next[j];
        }
        __syncthreads();
    }
    compute((n_k - 1) & 1);

    // epilogue: register r of lane l is out[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] of its tile
    if constexpr (!KSPLIT && !Q8) {
        if (a.img_kind) { // registers 4g .. 4g + 3: four consecutive rows (keys) of one column
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + wn * WN + j * 32 + r32;
                if (col >= a.n) continue;
                const float bj = a.bias ? a.bias[col] : 0.f;
                const int h = col / a.img_d, dim = col - h * a.img_d;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int row0 = m0 + wm * WM + i * 32 + 8 * g + 4 * (lane >> 5);
                        if (row0 >= a.m) continue;
                        const f32x4 v = {acc[i][j][4 * g] + bj, acc[i][j][4 * g + 1] + bj, acc[i][j][4 * g + 2] + bj,
                                         acc[i][j][4 * g + 3] + bj};
                        zwg_img::store_quad(a.img, a.img_kind, row0, h, dim, v, a.img_ctx, a.img_d, a.img_heads,
                                            a.img_tiles);
                    }
            }
            return;
        }
    }
    if constexpr (!KSPLIT) {
        const int rows_o = min(BM, a.m - m0);
        const int64_t span = (int64_t)(rows_o - 1) * a.ldo + (a.n - n0); // elements from (m0, n0) on
        if (a.epi == zwg_ew::kEpiAdd && span < 0x1fffffffll) {
            // out + v: each row block's residual values are loaded before its first store.  Loads
            // and stores interleaved per element (the compiler cannot move a load of out above a
            // store to out it cannot tell apart) would wait one memory round trip each.  The loads
            // go through a descriptor ending at the tile's last element (rows past m read 0), with
            // the lane's part of the offset in one VGPR and the register's row in the SGPR part.
            const __amdgpu_buffer_rsrc_t o_src = rsrc(a.out + (int64_t)m0 * a.ldo + n0, (uint32_t)(span * 4));
            const int ld4 = (int)a.ldo * 4;
            const int vo = (wm * WM + 4 * (lane >> 5)) * ld4 + (wn * WN + r32) * 4;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                float res[TN][16];
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        res[j][r] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(
                                       o_src, vo, (i * 32 + 8 * (r >> 2) + (r & 3)) * ld4 + j * 128, 0));
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int col = n0 + wn * WN + j * 32 + r32;
                    if (col >= a.n) continue;
                    const float bj = a.bias ? a.bias[col] : 0.f;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        if (row >= a.m) continue;
                        a.out[(int64_t)row * a.ldo + col] = res[j][r] + (acc[i][j][r] + bj);
                    }
                }
            }
            return;
        }
    }
    float *part = KSPLIT ? a.part + (int64_t)split * a.m * a.n : nullptr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + r32;
        if (col >= a.n) continue;
        const float bj = (!KSPLIT && a.bias) ? a.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= a.m) continue;
                if constexpr (KSPLIT) part[(int64_t)row * a.n + col] = acc[i][j][r];
                else if (a.epi == zwg_ew::kEpiAdd) // a residual spanning 2^31 bytes or more
                    zwg_ew::epilogue_store(&a.out[(int64_t)row * a.ldo + col], acc[i][j][r] + bj, a.epi);
                else {
                    // written once and not read again here: a non-temporal store keeps the x rows
                    // that the neighbouring column tiles re-read in L2
                    const float v = acc[i][j][r] + bj;
                    __builtin_nontemporal_store(a.epi == zwg_ew::kEpiGelu ? zwg_ew::gelu(v) : v,
                                                &a.out[(int64_t)row * a.ldo + col]);
                }
            }
    }
}

template <int BM, int BN, int WMODE, int NWN = 2, bool KSPLIT = false>
__global__ __launch_bounds__(128 * NWN) void linear_mfma_kernel(LinearArgs a) {
    linear_mfma_body<BM, BN, WMODE, NWN, KSPLIT>(a);
}

// KSPLIT launches n_split workgroups per tile (a.k_split, a.part set); otherwise n_split is 1
template <int BM, int BN, int WMODE, int NWN = 2, bool KSPLIT = false>
inline hipError_t launch_linear_tile(const LinearArgs &a, int n_split, hipStream_t stream) {
    const int64_t tiles = (int64_t)((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
    if (tiles > 0x7fffffffll || n_split < 1 || n_split > 65535 || (!KSPLIT && n_split != 1)) return hipErrorInvalidValue;
    linear_mfma_kernel<BM, BN, WMODE, NWN, KSPLIT><<<dim3((unsigned)tiles, (unsigned)n_split), 128 * NWN, 0, stream>>>(a);
    return hipGetLastError();
}

} // namespace zwg_lin
