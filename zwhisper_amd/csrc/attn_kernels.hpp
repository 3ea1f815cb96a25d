// Kernel arguments and launch entry points shared by the host layer (zw_gpu.hip) and the
// kernels (attn_flash.hip, attn_decode.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_geometry.hpp"

namespace zwg {

// Everything a kernel needs for one call, passed by value.  Counts are int32 (checked on
// the host), strides int64, all in floats.
struct AttnArgs {
    const float *q;
    const float *k;
    const float *v;
    float *out;
    int64_t q_stride, kv_stride, out_stride, kt_stride; // kt_stride 0: row-major K
    int64_t q_bstride, k_bstride, v_bstride, out_bstride;
    const int32_t *n_kv_item; // per-item key counts, or nullptr (then n_kv for all)
    int32_t n_q, n_kv, n_head, n_head_kv, group; // group = n_head / n_head_kv
    int32_t n_batch;
    int32_t causal;
    float scale_log2; // f32(1/sqrt(d)) * log2(e): scores go straight into exp2
    // split-KV (see unit_split)
    int32_t split_tile; // keys per tile of the split (the kernel's key tile)
    int32_t chunk_len;  // keys per split aimed at, a multiple of split_tile
    int32_t max_chunks; // partial slots per row; 1 = the kernel writes `out` itself
    int32_t heavy_first; // dense kernel: dispatch the longest (causal) q-blocks first
    int32_t xcd_group;   // dense kernel: run each head's q-blocks on one XCD (dense_unit)
    int32_t rows_per_unit; // query rows sharing one key range (flash: BM; decode: n_q)
    int64_t live_blocks;   // dense, heavy_first == 2: workgroups of the grid (dense_live_unit)
    float *part_o;      // [row][max_chunks][d]   unnormalised sum of p*v
    float *part_ml;     // [row][max_chunks][2]   (running max in log2 units, sum of p)
    // when set, the kernels that write `out` (the dense kernels' unsplit rows and the merge) raise
    // these words (kOutMaxSlots of them, out_max_record) to the largest |value| they write, as its
    // f32 bit pattern: an infinity or a NaN gives a pattern of 0x7f800000 or more
    uint32_t *out_max;
    // the dense x3 kernel only: K and V as tile images (kv_image.hpp) of img_tiles 32-key tiles per
    // (item, KV head), in place of k and v; null otherwise
    const _Float16 *k_img;
    const _Float16 *v_img;
    int32_t img_tiles;
    // the decode kernels only: when q_parts > 1, q holds the q_parts k-split partial sums of the
    // queries' projection, q_part_stride floats apart, and a query value is their sum in split
    // order plus q_bias[column] (load_q) -- the projection's split sum, taken in the q load
    int32_t q_parts;
    int64_t q_part_stride;
    const float *q_bias;
};

// Query value at float offset `at` of a.q, column `col` of its row (head * d + dim): a.q[at], or
// with q_parts > 1 (at most kMaxQParts) the projection's split sum formed here, as
// linear_split_sum_group_kernel forms it (partials added in split order, then the bias), so the
// value is the same bit for bit.  Every part's load goes out before the first add.
constexpr int kMaxQParts = 8;
__device__ __forceinline__ float load_q(const AttnArgs &a, int64_t at, int col) {
    if (a.q_parts <= 1) return a.q[at];
    float v[kMaxQParts];
#pragma unroll
    for (int j = 0; j < kMaxQParts; ++j)
        if (j < a.q_parts) v[j] = a.q[at + j * a.q_part_stride];
    float s = v[0];
#pragma unroll
    for (int j = 1; j < kMaxQParts; ++j)
        if (j < a.q_parts) s = s + v[j];
    return a.q_bias ? s + a.q_bias[col] : s;
}

// |x| as its bit pattern: for non-negative floats the unsigned order is the float order, and
// NaNs and infinities lie above every finite value.
__device__ __forceinline__ uint32_t abs_bits(float x) { return __builtin_bit_cast(uint32_t, x) & 0x7fffffffu; }

// The result maximum is kept in kOutMaxSlots words kOutMaxStride words (128 bytes) apart, and
// the host takes the largest: a merge launch of thousands of one-wave workgroups raising a single
// word serialises on it (measured 5.6 -> 39 us for a 3000-workgroup merge; with 32 slots 7.7 us,
// and neither 128 slots nor skipping the atomic when a read of the slot already shows as much
// measured faster).
constexpr int kOutMaxSlots = 32;
constexpr int kOutMaxStride = 32;
constexpr int kOutMaxBytes = kOutMaxSlots * kOutMaxStride * 4;

// Raise slot blockIdx.x % kOutMaxSlots of a.out_max to the wave's largest abs_bits `m` (one
// atomic per wave, its result unused).
__device__ __forceinline__ void out_max_record(const AttnArgs &a, uint32_t m) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
    if ((threadIdx.x & 63) == 0) atomicMax(a.out_max + (blockIdx.x % kOutMaxSlots) * kOutMaxStride, m);
}

// Rows of a call are numbered ((item * n_head + head) * n_q + query).
__host__ __device__ inline int64_t row_index(const AttnArgs &a, int item, int head, int query) {
    return ((int64_t)item * a.n_head + head) * a.n_q + query;
}

// Keys of batch item `item`: its own count when the call has per-item counts, clamped to the
// capacity n_kv the buffers were sized for.
__device__ inline int item_kv(const AttnArgs &a, int item) {
    return a.n_kv_item ? min(max(a.n_kv_item[item], 0), a.n_kv) : a.n_kv;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Decode grids over items with their own key counts (n_kv_item): the launch covers max_chunks
// chunks of every (item, KV head), but an item of few keys has fewer non-empty chunks.  MI355X
// deals consecutive workgroups round-robin over its XCDs and their CUs, so with the plain
// (item, chunk, KV head) order every CU would keep meeting the same chunk index: the CUs given the
// first chunks would stream full loads while those given the last ones sat idle.  Instead the
// workgroups are renumbered over the list of non-empty chunks, item by item (chunk, then KV head,
// fastest), so consecutive workgroups -- and so every CU -- get an even share; workgroups past the
// list's end exit.  Each wave computes the list from the key counts itself (items = lanes,
// kDecodeCompactItems at most).  Returns false for a workgroup past the end.
constexpr int kDecodeCompactItems = 256;
__device__ inline bool decode_compact_unit(const AttnArgs &a, int tile, int64_t wg, int *item, int *chunk, int *hk) {
    const int lane = (int)(threadIdx.x & 63);
    const int H = a.n_head_kv;
    int base = 0; // workgroups of the items before this lane group
#pragma unroll
    for (int k = 0; k < kDecodeCompactItems / 64; ++k) {
        const int it = lane + 64 * k;
        int c = 0;
        if (it < a.n_batch) {
            int ck;
            c = unit_split(item_kv(a, it), tile, a.chunk_len, a.max_chunks, &ck) * H;
        }
        int incl = c; // inclusive scan over the lanes
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off);
            if (lane >= off) incl += v;
        }
        const unsigned long long hit = __ballot(it < a.n_batch && base + incl > wg);
        if (hit) {
            const int first = __builtin_ctzll(hit);
            const int excl = base + __shfl(incl - c, first);
            const int local = (int)(wg - excl);
            *item = first + 64 * k;
            *chunk = local / H;
            *hk = local - *chunk * H;
            return true;
        }
        base += __shfl(incl, 63);
    }
    return false;
}

// Causal dense calls with one key count for every item (heavy_first == 2): the grid holds only the
// (q-block, chunk, item*head) triples that have keys -- a chunk index past its q-block's chunk
// count would leave a workgroup with nothing to do, scattered through the grid -- ranked longest
// q-block first, then chunk, with item*head fastest.  The hardware deals workgroup b to CU
// b mod 256, so each band of 256 ranks puts one workgroup on every CU; the odd bands are dealt in
// reverse (the CU given a band's heaviest workgroup gets the next band's lightest), which evens
// out each CU's total.  A partial last band keeps its order.
__device__ inline void dense_live_unit(const AttnArgs &a, int64_t lb, int n_qblocks, int bm, int bn, int *qb,
                                       int *chunk, int *ih) {
    const int64_t n_ih = (int64_t)a.n_batch * a.n_head;
    const int64_t band = lb >> 8;
    int64_t rank = lb;
    if ((band & 1) && (band + 1) * 256 <= (int64_t)gridDim.x) rank = (band << 8) + 255 - (lb & 255);
    int q = n_qblocks - 1;
    int n_ch = 1;
    for (; q > 0; --q) {
        const int q_end = min((q + 1) * bm, a.n_q);
        int ck;
        n_ch = unit_split(max(0, a.n_kv - a.n_q + q_end), bn, a.chunk_len, a.max_chunks, &ck);
        if (rank < (int64_t)n_ch * n_ih) break;
        rank -= (int64_t)n_ch * n_ih;
    }
    if (q == 0) {
        int ck;
        n_ch = unit_split(max(0, a.n_kv - a.n_q + min(bm, a.n_q)), bn, a.chunk_len, a.max_chunks, &ck);
    }
    *qb = q;
    *chunk = (int)(rank / n_ih);
    *ih = (int)(rank - (int64_t)*chunk * n_ih);
}

// MI355X deals consecutive workgroups round-robin over its 8 XCDs, each with its own L2.
// xcd_logical_block renumbers them so that consecutive logical ids run on the same XCD:
// hardware ids x, x+8, x+16, ... (all on XCD x) become one contiguous range of logical ids.
constexpr int kNumXCD = 8;
__device__ __forceinline__ int64_t xcd_logical_block(int64_t hw, int64_t n) {
    const int64_t xcd = hw % kNumXCD, local = hw / kNumXCD;
    const int64_t q = n / kNumXCD, r = n % kNumXCD;
    return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// Workgroup -> (item*head, q-block, chunk) of the dense kernels:
//  heavy_first 2  dense_live_unit (causal, one key count for every item)
//  heavy_first 1  ((n_qblocks - 1 - qb) * max_chunks + chunk) * n_batch*n_head + item*head: the
//                 longest (causal) q-blocks start first and shorter work fills the slots they
//                 free; heads vary fastest, so neighbouring workgroups -- which the hardware deals
//                 round-robin over the 8 XCDs -- carry equal work
//  otherwise      ((item*head) * n_qblocks + qb) * max_chunks + chunk, over xcd_logical_block when
//                 xcd_group is 1 (unsplit calls: a head's q-blocks share an XCD)
__device__ inline void dense_unit(const AttnArgs &a, int n_qblocks, int bm, int bn, int *qb, int *chunk, int *ih) {
    const int64_t lb = a.xcd_group ? xcd_logical_block(blockIdx.x, (int64_t)gridDim.x) : (int64_t)blockIdx.x;
    const int64_t n_ih = (int64_t)a.n_batch * a.n_head;
    if (a.heavy_first == 2) {
        dense_live_unit(a, lb, n_qblocks, bm, bn, qb, chunk, ih);
    } else if (a.heavy_first) {
        *ih = (int)(lb % n_ih);
        const int64_t t = lb / n_ih;
        *chunk = (int)(t % a.max_chunks);
        *qb = n_qblocks - 1 - (int)(t / a.max_chunks);
    } else {
        *chunk = (int)(lb % a.max_chunks);
        const int64_t lq = lb / a.max_chunks;
        *qb = (int)(lq % n_qblocks);
        *ih = (int)(lq / n_qblocks);
    }
}

hipError_t launch_flash(const AttnArgs &a, int d, hipStream_t stream, int *grid_blocks);
hipError_t launch_flash_x3(const AttnArgs &a, int d, hipStream_t stream, int *grid_blocks);
hipError_t launch_decode(const AttnArgs &a, int d, int rows, hipStream_t stream, int *grid_blocks);
hipError_t launch_combine(const AttnArgs &a, int d, hipStream_t stream);
// head dims above 128 (attn_generic.hip): any d % 4 == 0 up to kGenericMaxD, f32 on the VALU
constexpr int kGenericMaxD = 1024;
hipError_t launch_generic(const AttnArgs &a, int d, hipStream_t stream);
// head dims without kernels of their own (attn_pad.hip): zero-padded copies to the next built dim
hipError_t launch_pad_rows(const float *src, float *dst, int n_batch, int rows, int segs, int d, int D, int64_t srs,
                           int64_t sbs, const int32_t *n_rows_item, hipStream_t stream);
hipError_t launch_pad_kt(const float *src, float *dst, int n_batch, int n_head_kv, int d, int D, int kt, int n_kv,
                         int64_t sbs, const int32_t *n_kv_item, hipStream_t stream);
hipError_t launch_unpad_rows(const float *src, float *dst, int n_batch, int rows, int segs, int d, int D, int64_t drs,
                             int64_t dbs, hipStream_t stream);

typedef float lane_f32x2 __attribute__((ext_vector_type(2)));

// max / sum over lanes l and l ^ 32 (the two halves of a query's keys): v_permlane32_swap
// exchanges lanes 32..63 of its first register with lanes 0..31 of its second, so with x in both
// the two hold x of lanes 0..31 and of lanes 32..63 in every lane -- no LDS round trip.  Issued
// as inline asm: this compiler's __builtin_amdgcn_permlane32_swap returns the first register for
// both results.  The s_nop gives the two wait states the instruction needs after a VALU write of
// its operands.
__device__ __forceinline__ lane_f32x2 lane_halves(float x) {
    float a = x, b = x;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return (lane_f32x2){a, b};
}
__device__ __forceinline__ float lane_pair_max(float x) {
    const lane_f32x2 h = lane_halves(x);
    return fmaxf(h[0], h[1]);
}
__device__ __forceinline__ float lane_pair_sum(float x) {
    const lane_f32x2 h = lane_halves(x);
    return h[0] + h[1];
}

} // namespace zwg
