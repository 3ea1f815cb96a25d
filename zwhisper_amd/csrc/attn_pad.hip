// Head dims the attention kernels are not built for (any d % 4 == 0 up to 128, as the reference's
// d % V == 0, src/ops.zig:564): the call runs on the kernels of the next built dim D (32, 64 or
// 128) over copies of its tensors padded with zeros to D per head, and the result's first d dims
// of each head are copied back.  A zero dim adds exactly nothing to a score (q's padded dims are
// zero), and an output dim depends only on the same dim of V, so the first d dims equal the
// unpadded attention's.  The copies cost one extra read and write of each tensor; the built dims
// skip them.
#include <hip/hip_runtime.h>

#include "attn_kernels.hpp"

namespace zwg {

namespace {

constexpr int kPadThreads = 256;
constexpr int64_t kPadMaxBlocks = 1 << 20;

inline unsigned pad_blocks(int64_t n4) {
    const int64_t b = (n4 + kPadThreads - 1) / kPadThreads;
    return (unsigned)(b < kPadMaxBlocks ? (b > 0 ? b : 1) : kPadMaxBlocks);
}

// dst [b][r][s][D] <- src + b * sbs + r * srs + s * d, dims >= d and rows >= the item's row count
// set to zero; one thread per 4 floats (d, D, strides are multiples of 4)
__global__ __launch_bounds__(kPadThreads) void pad_rows_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                              int32_t n_batch, int32_t rows, int32_t segs, int32_t d,
                                                              int32_t D, int64_t srs, int64_t sbs,
                                                              const int32_t *n_rows_item) {
    const int64_t d4 = D / 4;
    const int64_t n4 = (int64_t)n_batch * rows * segs * d4;
    for (int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; f < n4; f += (int64_t)gridDim.x * blockDim.x) {
        const int j = 4 * (int)(f % d4);
        int64_t t = f / d4;
        const int s = (int)(t % segs);
        t /= segs;
        const int r = (int)(t % rows);
        const int b = (int)(t / rows);
        int live = rows;
        if (n_rows_item) live = min(max(n_rows_item[b], 0), rows);
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (j < d && r < live) v = *reinterpret_cast<const f32x4 *>(src + b * sbs + r * srs + (int64_t)s * d + j);
        *reinterpret_cast<f32x4 *>(dst + f * 4) = v;
    }
}

// transposed K: dst [b][hk][D][kt] <- rows hk * d + j of src + b * sbs (row stride kt) for j < d,
// columns past the item's key count and rows j >= d set to zero
__global__ __launch_bounds__(kPadThreads) void pad_kt_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                            int32_t n_batch, int32_t n_head_kv, int32_t d, int32_t D,
                                                            int32_t kt, int32_t n_kv, int64_t sbs,
                                                            const int32_t *n_kv_item) {
    const int64_t c4 = kt / 4;
    const int64_t n4 = (int64_t)n_batch * n_head_kv * D * c4;
    for (int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; f < n4; f += (int64_t)gridDim.x * blockDim.x) {
        const int c = 4 * (int)(f % c4);
        int64_t t = f / c4;
        const int j = (int)(t % D);
        t /= D;
        const int hk = (int)(t % n_head_kv);
        const int b = (int)(t / n_head_kv);
        int live = n_kv;
        if (n_kv_item) live = min(max(n_kv_item[b], 0), n_kv);
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (j < d) {
            const float *row = src + b * sbs + ((int64_t)hk * d + j) * kt;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (c + e < live) v[e] = row[c + e];
        }
        *reinterpret_cast<f32x4 *>(dst + f * 4) = v;
    }
}

// out + b * dbs + r * drs + s * d <- the first d dims of src [b][r][s][D]
__global__ __launch_bounds__(kPadThreads) void unpad_rows_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                                int32_t n_batch, int32_t rows, int32_t segs, int32_t d,
                                                                int32_t D, int64_t drs, int64_t dbs) {
    const int64_t d4 = d / 4;
    const int64_t n4 = (int64_t)n_batch * rows * segs * d4;
    for (int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; f < n4; f += (int64_t)gridDim.x * blockDim.x) {
        const int j = 4 * (int)(f % d4);
        int64_t t = f / d4;
        const int s = (int)(t % segs);
        t /= segs;
        const int r = (int)(t % rows);
        const int b = (int)(t / rows);
        const f32x4 v = *reinterpret_cast<const f32x4 *>(src + ((t * segs + s) * D) + j);
        *reinterpret_cast<f32x4 *>(dst + b * dbs + r * drs + (int64_t)s * d + j) = v;
    }
}

} // namespace

hipError_t launch_pad_rows(const float *src, float *dst, int n_batch, int rows, int segs, int d, int D, int64_t srs,
                           int64_t sbs, const int32_t *n_rows_item, hipStream_t stream) {
    const int64_t n4 = (int64_t)n_batch * rows * segs * (D / 4);
    if (n4 == 0) return hipSuccess;
    pad_rows_kernel<<<pad_blocks(n4), kPadThreads, 0, stream>>>(src, dst, n_batch, rows, segs, d, D, srs, sbs,
                                                                n_rows_item);
    return hipGetLastError();
}

hipError_t launch_pad_kt(const float *src, float *dst, int n_batch, int n_head_kv, int d, int D, int kt, int n_kv,
                         int64_t sbs, const int32_t *n_kv_item, hipStream_t stream) {
    const int64_t n4 = (int64_t)n_batch * n_head_kv * D * (kt / 4);
    if (n4 == 0) return hipSuccess;
    pad_kt_kernel<<<pad_blocks(n4), kPadThreads, 0, stream>>>(src, dst, n_batch, n_head_kv, d, D, kt, n_kv, sbs,
                                                              n_kv_item);
    return hipGetLastError();
}

hipError_t launch_unpad_rows(const float *src, float *dst, int n_batch, int rows, int segs, int d, int D, int64_t drs,
                             int64_t dbs, hipStream_t stream) {
    const int64_t n4 = (int64_t)n_batch * rows * segs * (d / 4);
    if (n4 == 0) return hipSuccess;
    unpad_rows_kernel<<<pad_blocks(n4), kPadThreads, 0, stream>>>(src, dst, n_batch, rows, segs, d, D, drs, dbs);
    return hipGetLastError();
}

} // namespace zwg
