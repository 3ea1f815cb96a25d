// Split-K streaming attention for few query rows per KV head (token-at-a-time decode).
//
// The reference runs single-token decode through the same (head, q-block) task as prefill
// (AttnJob.run, src/ops.zig:517-541, called at n_q = 1 from src/decoder.zig:184, :191 and
// src/llm.zig:191-202), which re-reads KT and V once per query head.  Here one workgroup takes
// one (item, KV head, key chunk) and carries every query row that shares that KV head
// (heads of the GQA group x queries, at most kDecodeMaxRows), so each K/V byte is read from
// HBM once.  The chunk is walked in 256-key tiles with an online softmax; the partial
// (max, sum, sum of p*v) of each row and chunk goes to the workspace and combine_kernel
// merges the chunks, or the block writes the output itself when a row has one chunk.
//
// Scores: transposed K ([d][stride] per KV head) is read with lanes along keys (16-byte
// loads of 4 keys, wave reads 1 KB contiguous per dim); row-major K ([key][stride]) with
// D/4 lanes per key row (one 16-byte load each) and a cross-lane sum.  V is row-major in
// every caller: D/4 lanes per key row, each lane accumulating 4 dims of every row.
#include "attn_kernels.hpp"

namespace zwg {

static __device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

static __device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
static __device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <int D, int R, bool KT>
__global__ __launch_bounds__(kDecodeThreads) void decode_attn_kernel(AttnArgs a) {
    constexpr int T = kDecodeTile;
    constexpr int L = D / 4;            // lanes per key row (row-major loads)
    constexpr int P = kDecodeThreads / L; // key rows per pass
    constexpr int NP = T / P;           // passes over a tile's key rows
    // loads in flight per thread: 16, or 8 when many rows multiply the operands held with them
    constexpr int MAXB = R > 2 ? 8 : 16;
    constexpr int PB = NP < MAXB ? NP : MAXB; // key/value row loads per batch
    constexpr int DK = D / 4;           // dims per dim group (transposed K)
    constexpr int KB = DK < MAXB ? DK : MAXB; // transposed-K loads per batch
    constexpr int RED = KT ? 4 * R * T : 4 * R * D;
    static_assert(4 * R * D <= RED, "reduction buffer too small");

    __shared__ __align__(16) float q_s[R][D];
    __shared__ __align__(16) float s_s[R][T];
    __shared__ __align__(16) float red[RED];
    __shared__ float alpha_s[R], m_s[R], l_s[R];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int chunk = blockIdx.x;
    const int hk = blockIdx.y;
    const int item = blockIdx.z;

    const int n_q = a.n_q;
    const int G = a.group;
    const int rows = n_q * G;
    const int n_kv = item_kv(a, item);
    // the last query sees every key, so the unit's key range is [0, n_kv)
    const int n_chunks = max(1, (n_kv + a.chunk_len - 1) / a.chunk_len);
    if (chunk >= n_chunks) return;
    const int k_begin = chunk * a.chunk_len;
    const int k_end = min(n_kv, k_begin + a.chunk_len);
    const int diag = n_kv - n_q;

    // row r = query (r / G) of head hk*G + r % G
    for (int idx = tid; idx < R * D; idx += kDecodeThreads) {
        const int r = idx / D;
        const int p = idx - r * D;
        float val = 0.f;
        if (r < rows) {
            const int qi = r / G;
            const int head = hk * G + (r - qi * G);
            val = a.q[item * a.q_bstride + (int64_t)qi * a.q_stride + head * D + p] * a.scale_log2;
        }
        q_s[r][p] = val;
    }
    if (tid < R) {
        m_s[tid] = -INFINITY;
        l_s[tid] = 0.f;
    }
    __syncthreads();

    const int c = tid % L;     // this thread's 4 dims: 4c .. 4c+3
    const int kslot = tid / L; // this thread's key row within a pass
    float qr[R][4];
    if (!KT) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) qr[r][i] = q_s[r][4 * c + i];
    }
    float o[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[r][i] = 0.f;

    const float *kbase = a.k + item * a.k_bstride + (KT ? (int64_t)hk * D * a.kt_stride : (int64_t)hk * D);
    const float *vbase = a.v + item * a.v_bstride + hk * D + 4 * c;

    for (int k0 = k_begin; k0 < k_end; k0 += T) {
        const int kn = min(T, k_end - k0);
        // ---- scores of this tile into s_s (log2 units)
        if (KT) {
            const int kq = tid & 63;
            const int dg = tid >> 6;
            float acc[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[r][i] = 0.f;
            if (4 * kq < kn) {
                // k0 + 4kq < n_kv <= kt_stride and kt_stride % 4 == 0: the 16-byte load is in bounds
                const float *kp = kbase + (int64_t)(dg * DK) * a.kt_stride + k0 + 4 * kq;
#pragma unroll 1
                for (int p0 = 0; p0 < DK; p0 += KB) {
                    // issue the whole batch of loads before using any of them
                    float4 kk[KB];
#pragma unroll
                    for (int i = 0; i < KB; ++i)
                        kk[i] = *reinterpret_cast<const float4 *>(kp + (int64_t)(p0 + i) * a.kt_stride);
#pragma unroll
                    for (int i = 0; i < KB; ++i)
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const float qv = q_s[r][dg * DK + p0 + i];
                            acc[r][0] += qv * kk[i].x;
                            acc[r][1] += qv * kk[i].y;
                            acc[r][2] += qv * kk[i].z;
                            acc[r][3] += qv * kk[i].w;
                        }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
                *reinterpret_cast<float4 *>(&red[(dg * R + r) * T + 4 * kq]) =
                    make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
            __syncthreads();
            for (int idx = tid; idx < R * T; idx += kDecodeThreads) {
                const int r = idx / T;
                const int j = idx - r * T;
                s_s[r][j] = red[(0 * R + r) * T + j] + red[(1 * R + r) * T + j] + red[(2 * R + r) * T + j] +
                            red[(3 * R + r) * T + j];
            }
        } else {
#pragma unroll 1
            for (int b0 = 0; b0 < NP; b0 += PB) {
                float4 kk[PB];
#pragma unroll
                for (int i = 0; i < PB; ++i) {
                    const int j = kslot + (b0 + i) * P;
                    kk[i] = j < kn ? *reinterpret_cast<const float4 *>(kbase + (int64_t)(k0 + j) * a.kv_stride + 4 * c)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int i = 0; i < PB; ++i) {
                    const int j = kslot + (b0 + i) * P;
                    float part[R];
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        part[r] = qr[r][0] * kk[i].x + qr[r][1] * kk[i].y + qr[r][2] * kk[i].z + qr[r][3] * kk[i].w;
#pragma unroll
                    for (int off = L / 2; off >= 1; off >>= 1)
#pragma unroll
                        for (int r = 0; r < R; ++r) part[r] += __shfl_xor(part[r], off);
                    if (c == 0) {
#pragma unroll
                        for (int r = 0; r < R; ++r) s_s[r][j] = part[r];
                    }
                }
            }
        }
        __syncthreads();
        // ---- mask, online softmax; wave w owns rows w, w + 4
        for (int r = wave; r < R; r += 4) {
            int vlim = 0;
            if (r < rows) vlim = min(kn, (a.causal ? diag + r / G + 1 : n_kv) - k0);
            float v[T / 64];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < T / 64; ++i) {
                const int j = lane + 64 * i;
                v[i] = j < vlim ? s_s[r][j] : -INFINITY;
                mx = fmaxf(mx, v[i]);
            }
            mx = wave_max(mx);
            const float m_old = m_s[r];
            const float m_new = fmaxf(m_old, mx);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < T / 64; ++i) {
                const float p = exp2_fast(v[i] - m_use);
                s_s[r][lane + 64 * i] = p;
                sum += p;
            }
            sum = wave_sum(sum);
            if (lane == 0) {
                const float alpha = exp2_fast(m_old - m_use);
                alpha_s[r] = alpha;
                l_s[r] = l_s[r] * alpha + sum;
                m_s[r] = m_new;
            }
        }
        __syncthreads();
        // ---- o += p . V
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float al = alpha_s[r];
#pragma unroll
            for (int i = 0; i < 4; ++i) o[r][i] *= al;
        }
#pragma unroll 1
        for (int b0 = 0; b0 < NP; b0 += PB) {
            float4 vv[PB];
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const int j = kslot + (b0 + i) * P;
                vv[i] = j < kn ? *reinterpret_cast<const float4 *>(vbase + (int64_t)(k0 + j) * a.kv_stride)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const int j = kslot + (b0 + i) * P;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float p = s_s[r][j];
                    o[r][0] += p * vv[i].x;
                    o[r][1] += p * vv[i].y;
                    o[r][2] += p * vv[i].z;
                    o[r][3] += p * vv[i].w;
                }
            }
        }
        __syncthreads();
    }

    // ---- sum o over the key rows: lanes L apart within a wave, then the 4 waves through LDS
#pragma unroll
    for (int off = L; off < 64; off <<= 1)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[r][i] += __shfl_xor(o[r][i], off);
    if (lane < L) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            *reinterpret_cast<float4 *>(&red[(wave * R + r) * D + 4 * c]) = make_float4(o[r][0], o[r][1], o[r][2], o[r][3]);
    }
    __syncthreads();
    for (int idx = tid; idx < R * D; idx += kDecodeThreads) {
        const int r = idx / D;
        const int p = idx - r * D;
        if (r >= rows) continue;
        const float acc = red[(0 * R + r) * D + p] + red[(1 * R + r) * D + p] + red[(2 * R + r) * D + p] +
                          red[(3 * R + r) * D + p];
        const int qi = r / G;
        const int head = hk * G + (r - qi * G);
        if (a.max_chunks == 1) {
            const float l = l_s[r];
            a.out[item * a.out_bstride + (int64_t)qi * a.out_stride + head * D + p] = l > 0.f ? acc / l : 0.f;
        } else {
            const int64_t slot = row_index(a, item, head, qi) * a.max_chunks + chunk;
            a.part_o[slot * D + p] = acc;
            if (p == 0) {
                a.part_ml[2 * slot] = m_s[r];
                a.part_ml[2 * slot + 1] = l_s[r];
            }
        }
    }
}

hipError_t launch_decode(const AttnArgs &a, int d, int rows, hipStream_t stream, int *grid_blocks) {
    dim3 grid(a.max_chunks, a.n_head_kv, a.n_batch);
    dim3 block(kDecodeThreads);
    if (grid_blocks) *grid_blocks = (int)(grid.x * grid.y * grid.z);
    const bool kt = a.kt_stride != 0;
    const int R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : rows <= 6 ? 6 : 8;
    if (rows > kDecodeMaxRows) return hipErrorInvalidValue;
#define ZWG_DEC(DD, RR)                                                                                          \
    if (kt)                                                                                                      \
        decode_attn_kernel<DD, RR, true><<<grid, block, 0, stream>>>(a);                                         \
    else                                                                                                         \
        decode_attn_kernel<DD, RR, false><<<grid, block, 0, stream>>>(a);
#define ZWG_DEC_R(DD)                                                                                            \
    switch (R) {                                                                                                 \
    case 1: ZWG_DEC(DD, 1); break;                                                                               \
    case 2: ZWG_DEC(DD, 2); break;                                                                               \
    case 4: ZWG_DEC(DD, 4); break;                                                                               \
    case 6: ZWG_DEC(DD, 6); break;                                                                               \
    default: ZWG_DEC(DD, 8); break;                                                                              \
    }
    switch (d) {
    case 32: ZWG_DEC_R(32); break;
    case 64: ZWG_DEC_R(64); break;
    case 128: ZWG_DEC_R(128); break;
    default: return hipErrorInvalidValue;
    }
#undef ZWG_DEC_R
#undef ZWG_DEC
    return hipGetLastError();
}

} // namespace zwg
