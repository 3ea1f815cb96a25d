// Head dims above the built kernels' 128 (the reference takes any d % V == 0, src/ops.zig:564;
// this kernel any d % 4 == 0 up to kGenericMaxD): one wavefront per (item, head, query) row, in
// plain f32 on the VALU.  None of zwhisper's models has such a head dim, so this is the path that
// keeps the drop-in whole, not a tuned one.
//
//   q row in LDS (pre-scaled into log2 units); keys in tiles of 64, lane j scoring key k0 + j with
//   the whole row's dot product (float4 loads of its K row, or of the transposed K's columns);
//   causal and key-count masking; the online softmax (tile max over the wave, exp2, lazily moved
//   running max as in the other kernels); then O += P . V with lane l owning dims l, l + 64, ...,
//   reading each value row's dims across the lanes (coalesced) and each p by a lane shuffle.
//   The row is written normalised, as the reference writes its output rows (src/ops.zig:540).
#include <hip/hip_runtime.h>

#include "attn_kernels.hpp"

namespace zwg {

namespace {

constexpr int kGenericWaves = 4;

template <int DP> // dims per lane in the P.V accumulation: d <= 64 * DP
__global__ __launch_bounds__(64 * kGenericWaves) void attn_generic_kernel(AttnArgs a, int32_t d) {
    __shared__ __align__(16) float q_s[kGenericWaves][64 * DP];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n_rows = (int64_t)a.n_batch * a.n_head * a.n_q;
    // (item * n_head + head) * n_q + query; the last workgroup's spare waves take the last row,
    // compute it and do not store it
    const int64_t row_w = (int64_t)blockIdx.x * kGenericWaves + wave;
    const bool live = row_w < n_rows;
    const int64_t row = live ? row_w : n_rows - 1;
    const int query = (int)(row % a.n_q);
    const int64_t ih = row / a.n_q;
    const int head = (int)(ih % a.n_head);
    const int item = (int)(ih / a.n_head);
    const int hk = head / a.group;
    const int n_kv = item_kv(a, item);
    const int lim = a.causal ? min(n_kv, n_kv - a.n_q + query + 1) : n_kv; // keys this row sees

    const float *qp = a.q + item * a.q_bstride + (int64_t)query * a.q_stride + (int64_t)head * d;
    float *qs = q_s[wave];
    for (int p = lane; p < d; p += 64) qs[p] = qp[p] * a.scale_log2;
    __syncthreads();

    const float *kbase = a.k + item * a.k_bstride + (a.kt_stride ? (int64_t)hk * d * a.kt_stride : (int64_t)hk * d);
    const float *vbase = a.v + item * a.v_bstride + (int64_t)hk * d;
    float o[DP];
#pragma unroll
    for (int e = 0; e < DP; ++e) o[e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    for (int k0 = 0; k0 < lim; k0 += 64) {
        const int key = k0 + lane;
        float s = -INFINITY;
        if (key < lim) {
            float acc = 0.f;
            if (a.kt_stride) {
                const float *kc = kbase + key;
                for (int p = 0; p < d; ++p) acc = __builtin_fmaf(qs[p], kc[(int64_t)p * a.kt_stride], acc);
            } else {
                const float4 *kr = reinterpret_cast<const float4 *>(kbase + (int64_t)key * a.kv_stride);
                for (int p4 = 0; p4 < d / 4; ++p4) {
                    const float4 kk = kr[p4];
                    acc = __builtin_fmaf(qs[4 * p4], kk.x, acc);
                    acc = __builtin_fmaf(qs[4 * p4 + 1], kk.y, acc);
                    acc = __builtin_fmaf(qs[4 * p4 + 2], kk.z, acc);
                    acc = __builtin_fmaf(qs[4 * p4 + 3], kk.w, acc);
                }
            }
            s = acc;
        }
        float mt = s;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off));
        if (mt > m_run + 8.0f || m_run == -INFINITY) { // the running max moves (wave-uniform)
            const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mt);
            l_run *= alpha;
#pragma unroll
            for (int e = 0; e < DP; ++e) o[e] *= alpha;
            m_run = fmaxf(m_run, mt);
        }
        const float pj = key < lim ? __builtin_amdgcn_exp2f(s - m_run) : 0.f;
        float ls = pj;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ls += __shfl_xor(ls, off);
        l_run += ls;
        const int n_t = min(64, lim - k0);
        for (int j = 0; j < n_t; ++j) {
            const float pjj = __shfl(pj, j);
            const float *vr = vbase + (int64_t)(k0 + j) * a.kv_stride;
#pragma unroll
            for (int e = 0; e < DP; ++e) {
                const int dim = lane + 64 * e;
                if (dim < d) o[e] = __builtin_fmaf(pjj, vr[dim], o[e]);
            }
        }
    }
    if (!live) return;
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    float *op = a.out + item * a.out_bstride + (int64_t)query * a.out_stride + (int64_t)head * d;
#pragma unroll
    for (int e = 0; e < DP; ++e) {
        const int dim = lane + 64 * e;
        if (dim < d) op[dim] = o[e] * inv;
    }
}

} // namespace

hipError_t launch_generic(const AttnArgs &a, int d, hipStream_t stream) {
    const int64_t rows = (int64_t)a.n_batch * a.n_head * a.n_q;
    const int64_t blocks = (rows + kGenericWaves - 1) / kGenericWaves;
    if (blocks > 0x7fffffffll || d % 4 != 0 || d > kGenericMaxD) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks), block(64 * kGenericWaves);
    if (d <= 256) attn_generic_kernel<4><<<grid, block, 0, stream>>>(a, d);
    else if (d <= 512) attn_generic_kernel<8><<<grid, block, 0, stream>>>(a, d);
    else attn_generic_kernel<16><<<grid, block, 0, stream>>>(a, d);
    return hipGetLastError();
}

} // namespace zwg
