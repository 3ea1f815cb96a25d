// The linear-layer kernel on gfx950 MFMA: out[i][o] = sum_p x[i][p] * w[o][p] (+ b[o]), x f32,
// w f16, out f32 (ops.linear with f16 weights, src/ops.zig:283-306, src/gemm.zig:117-137).
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
// Bounds.  Loads go through buffer descriptors whose range ends at the workgroup's last row of
// x (or w): rows past m (or n) read as 0 in hardware, and a K column past k gets an offset
// beyond the range, so the loop body has no branches.  The host guarantees k % 8 == 0 and a
// per-workgroup range below 2^31 bytes.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace zwg_lin {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int BK = 32;                 // K per LDS stage: one 64-byte LDS row
constexpr uint32_t kOutOfRange = 0x80000000u; // a buffer offset past every range the host allows

struct LinearArgs {
    const float *x;    // [m][ldx]
    const _Float16 *w; // [n][ldw]
    const float *bias; // [n] or nullptr
    float *out;        // [m][ldo]
    int64_t ldx, ldw, ldo;
    int32_t m, n, k;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

// half index of (row, 8-half chunk) in a swizzled LDS tile
__device__ __forceinline__ int lds_at(int row, int chunk) { return row * BK + ((chunk ^ ((row ^ (row >> 2)) & 3)) << 3); }

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void linear_f16_kernel(LinearArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2;   // per wave
    constexpr int TM = WM / 32, TN = WN / 32; // 32 x 32 MFMA tiles per wave
    constexpr int XL = BM * BK / 4 / kThreads; // float4 loads of x per thread per stage
    constexpr int WL = BN * BK / 8 / kThreads; // 8-half loads of w per thread per stage
    static_assert(XL >= 1 && WL >= 1 && TM >= 1 && TN >= 1, "tile too small for the workgroup");

    __shared__ __align__(16) _Float16 xh[2][BM * BK];
    __shared__ __align__(16) _Float16 xl[2][BM * BK];
    __shared__ __align__(16) _Float16 ws[2][BN * BK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;

    const int rows_x = min(BM, a.m - m0), rows_w = min(BN, a.n - n0);
    const __amdgpu_buffer_rsrc_t xr_src = rsrc(a.x + (int64_t)m0 * a.ldx, (uint32_t)(rows_x * a.ldx * 4));
    const __amdgpu_buffer_rsrc_t wr_src = rsrc(a.w + (int64_t)n0 * a.ldw, (uint32_t)(rows_w * a.ldw * 2));

    f32x4 xr[XL];
    half8 wr[WL];
    // stage loads: x element (row, 4 k) and w element (row, 8 k)
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
            const int row = f / (BK / 8), gk = k0 + 8 * (f % (BK / 8));
            const uint32_t off = gk < a.k ? (uint32_t)(row * a.ldw + gk) * 2u : kOutOfRange;
            wr[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(wr_src, (int)off, 0, 0));
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
            const int row = f / (BK / 8), c = f % (BK / 8);
            *reinterpret_cast<half8 *>(&ws[buf][lds_at(row, c)]) = wr[i];
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (f32x16){0};

    const int r32 = lane & 31, ch = lane >> 5;
    auto compute = [&](int buf) {
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
    };

    const int n_k = (a.k + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    for (int t = 0; t + 1 < n_k; ++t) {
        load((t + 1) * BK);
        compute(t & 1);
        store((t + 1) & 1);
        __syncthreads();
    }
    compute((n_k - 1) & 1);

    // epilogue: register r of lane l is out[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] of its tile
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 32 + r32;
        if (col >= a.n) continue;
        const float bj = a.bias ? a.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < a.m) a.out[(int64_t)row * a.ldo + col] = acc[i][j][r] + bj;
            }
    }
}

template <int BM, int BN>
inline hipError_t launch_linear_tile(const LinearArgs &a, hipStream_t stream) {
    dim3 grid((unsigned)((a.m + BM - 1) / BM), (unsigned)((a.n + BN - 1) / BN));
    linear_f16_kernel<BM, BN><<<grid, kThreads, 0, stream>>>(a);
    return hipGetLastError();
}

} // namespace zwg_lin
