// Split-K streaming attention for few query rows per KV head (token-at-a-time decode).
//
// The reference runs single-token decode through the same (head, q-block) task as prefill
// (AttnJob.run, src/ops.zig:517-541, called at n_q = 1 from src/decoder.zig:184, :191 and
// src/llm.zig:191-202), which re-reads KT and V once per query head.  Here a work unit is one
// (item, KV head) and carries every query row that shares that KV head (heads of the GQA group
// x queries, at most kDecodeMaxRows), so each K/V byte is read from HBM once.  A unit's keys
// are split into chunks; each chunk writes a partial (max, sum, sum of p*v) per row for
// combine_kernel, or the normalised output itself when its unit has a single chunk.
//
// Two kernels, by key layout:
//
// decode_kt_kernel -- transposed K ([d][kt_stride] per KV head, the LLM cache, src/llm.zig:27).
//   One wavefront per chunk, no workgroup barrier.  Each lane owns 4 consecutive keys of a
//   256-key step and forms their full dot products in-lane (16-byte loads, the wave reads 1 KB
//   contiguous per dim); the softmax is online per row; the step's probabilities go through a
//   wave-private LDS row to the V pass, where lanes run along the head dims.
//
// decode_rm_kernel -- row-major K ([key][kv_stride], the Whisper decoder caches,
//   src/decoder.zig:39-42).  One 256-thread workgroup per chunk, walked in tiles of T keys
//   (256, or 64 for caches of at most 512 keys, so short caches still split over many chunks):
//   D/4 lanes per key row with a butterfly sum for the scores, the tile's softmax in LDS, then
//   D/4 lanes per V row; loads are issued in batches so a thread has several in flight.
//
// With per-item key counts (n_kv_item) both kernels number their workgroups over the list of
// non-empty chunks (decode_compact_unit), so the CUs share the work evenly however the counts
// differ.
#include "attn_kernels.hpp"

namespace zwg {

static __device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Raw buffer loads: 32-bit byte offsets from a descriptor's base, split into a per-lane part
// (VGPR) and a wave-uniform part (SGPR), range-checked by the hardware against `bytes` (a load
// past it returns 0).
static __device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, (int)bytes, 0x00020000);
}
// The K/V caches are read once per step: every cache load is non-temporal (cache policy nt, bit 1
// of the buffer instruction's policy operand), which lets the stream pass the caches without
// displacing lines and, measured on this MI355X, raises a plain streaming read from 6.1 to
// 7.0 TB/s.
constexpr int kCachePolicyNT = 2;
static __device__ __forceinline__ f32x4 load_f32x4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kCachePolicyNT));
}
static __device__ __forceinline__ float4 load_nt(const float *p) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
}

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

#ifndef ZWG_DECODE_BATCH
#define ZWG_DECODE_BATCH 8
#endif

template <int D, int R>
__global__ __launch_bounds__(64) void decode_kt_kernel(AttnArgs a) {
    constexpr int T = kDecodeTile; // keys per step of the transposed-K path (64 lanes x 4)
    static_assert(T == 256, "the transposed-K step is 64 lanes x 4 keys");
    constexpr int L = D / 4;       // lanes per key row (row-major K and V)
    constexpr int G4 = 64 / L;     // key rows per wave instruction
    constexpr int NB = ZWG_DECODE_BATCH; // loads in flight per lane and per tensor

    __shared__ __align__(16) float q_s[R][D];
    __shared__ __align__(16) float p_s[R][T];

    const int lane = threadIdx.x;
    // one wave per (item, chunk, KV head), KV head fastest; over the non-empty chunks only when the
    // items have their own key counts (decode_compact_unit)
    int hk, chunk, item;
    if (a.n_kv_item && a.n_batch <= kDecodeCompactItems) {
        if (!decode_compact_unit(a, T, blockIdx.x, &item, &chunk, &hk)) return;
    } else {
        hk = blockIdx.x % a.n_head_kv;
        chunk = (blockIdx.x / a.n_head_kv) % a.max_chunks;
        item = blockIdx.x / (a.n_head_kv * a.max_chunks);
    }

    const int n_q = a.n_q;
    const int G = a.group;
    const int rows = n_q * G;
    // row r = query (r / G) of head hk*G + r % G; q pre-scaled into log2 units.  Staged before the
    // item's key count is read, so the two round trips overlap (a wave with no keys in its chunk
    // then drops its copy).
    for (int idx = lane; idx < R * D; idx += 64) {
        const int r = idx / D;
        const int p = idx - r * D;
        float val = 0.f;
        if (r < rows) {
            const int qi = r / G;
            const int head = hk * G + (r - qi * G);
            val = load_q(a, item * a.q_bstride + (int64_t)qi * a.q_stride + head * D + p, head * D + p) * a.scale_log2;
        }
        q_s[r][p] = val;
    }
    const int n_kv = item_kv(a, item);
    // the last query sees every key, so the unit's key range is [0, n_kv)
    int chunk_keys;
    const int n_chunks = unit_split(n_kv, T, a.chunk_len, a.max_chunks, &chunk_keys);
    if (chunk >= n_chunks) return;
    const int k_begin = chunk * chunk_keys;
    const int k_end = min(n_kv, k_begin + chunk_keys);
    const int diag = n_kv - n_q; // query i sees keys j <= diag + i
    __syncthreads();

    // exclusive key limit of each row: the chunk end, and the causal diagonal
    int lim[R];
#pragma unroll
    for (int r = 0; r < R; ++r) lim[r] = r < rows ? min(k_end, a.causal ? diag + r / G + 1 : n_kv) : 0;

    float m[R], l[R], o[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
        o[r][0] = o[r][1] = o[r][2] = o[r][3] = 0.f;
    }

    const float *kbase = a.k + item * a.k_bstride + (int64_t)hk * D * a.kt_stride;
    const float *vbase = a.v + item * a.v_bstride + hk * D;
    const int c = lane % L;  // this lane's dims in the V pass: 4c .. 4c+3
    const int grp = lane / L; // this lane's key row within an instruction

    {
        constexpr int KB = NB;
        constexpr int KEYS_PER_GRP = T / G4; // V pass: each lane group walks its own key range
#pragma unroll 1
        for (int k0 = k_begin; k0 < k_end; k0 += T) {
            float acc[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0.f;
            if (k0 + 4 * lane < k_end) {
                // k0 + 4*lane < n_kv <= kt_stride and kt_stride % 4 == 0: the 16-byte load is in bounds
                const float *kp = kbase + k0 + 4 * lane;
#pragma unroll 1
                for (int p0 = 0; p0 < D; p0 += KB) {
                    float4 kk[KB];
#pragma unroll
                    for (int i = 0; i < KB; ++i)
                        kk[i] = load_nt(kp + (int64_t)(p0 + i) * a.kt_stride);
#pragma unroll
                    for (int i = 0; i < KB; ++i)
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const float qv = q_s[r][p0 + i];
                            acc[r][0] += qv * kk[i].x;
                            acc[r][1] += qv * kk[i].y;
                            acc[r][2] += qv * kk[i].z;
                            acc[r][3] += qv * kk[i].w;
                        }
                }
            }
            float alpha[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s[4];
                float mx = -INFINITY;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s[i] = k0 + 4 * lane + i < lim[r] ? acc[r][i] : -INFINITY;
                    mx = fmaxf(mx, s[i]);
                }
                mx = wave_max(mx);
                const float m_new = fmaxf(m[r], mx);
                const float m_use = m_new == -INFINITY ? 0.f : m_new;
                alpha[r] = exp2_fast(m[r] - m_use);
                float4 p;
                p.x = exp2_fast(s[0] - m_use);
                p.y = exp2_fast(s[1] - m_use);
                p.z = exp2_fast(s[2] - m_use);
                p.w = exp2_fast(s[3] - m_use);
                l[r] = l[r] * alpha[r] + (p.x + p.y + p.z + p.w); // this lane's keys only
                m[r] = m_new;
                *reinterpret_cast<float4 *>(&p_s[r][4 * lane]) = p;
            }
            __syncthreads(); // single-wave block: orders the p_s writes before the reads below
#pragma unroll
            for (int r = 0; r < R; ++r) {
                o[r][0] *= alpha[r];
                o[r][1] *= alpha[r];
                o[r][2] *= alpha[r];
                o[r][3] *= alpha[r];
            }
            // lane group grp walks keys [grp*KEYS_PER_GRP, (grp+1)*KEYS_PER_GRP) of the step
            const int j_lo = grp * KEYS_PER_GRP;
            const int kn = min(T, k_end - k0);
#pragma unroll 1
            for (int j0 = 0; j0 < KEYS_PER_GRP; j0 += NB) {
                float4 vv[NB];
#pragma unroll
                for (int i = 0; i < NB; ++i) {
                    const int j = j_lo + j0 + i;
                    vv[i] = j < kn ? load_nt(vbase + (int64_t)(k0 + j) * a.kv_stride + 4 * c)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int i4 = 0; i4 < NB; i4 += 4) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float4 p = *reinterpret_cast<const float4 *>(&p_s[r][j_lo + j0 + i4]);
                        const float pp[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            o[r][0] += pp[u] * vv[i4 + u].x;
                            o[r][1] += pp[u] * vv[i4 + u].y;
                            o[r][2] += pp[u] * vv[i4 + u].z;
                            o[r][3] += pp[u] * vv[i4 + u].w;
                        }
                    }
                }
            }
            __syncthreads(); // before the next step overwrites p_s
        }
        // l: each lane summed its own keys; o: each lane group its own keys
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) l[r] += __shfl_xor(l[r], off);
#pragma unroll
            for (int off = L; off < 64; off <<= 1)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[r][i] += __shfl_xor(o[r][i], off);
        }
    }

    // lanes 0..L-1 hold rows' o for dims 4c..4c+3 (every lane group holds the same sums)
    if (lane >= L) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r >= rows) break;
        const int qi = r / G;
        const int head = hk * G + (r - qi * G);
        if (n_chunks == 1) {
            const float inv = l[r] > 0.f ? 1.f / l[r] : 0.f;
            float *op = a.out + item * a.out_bstride + (int64_t)qi * a.out_stride + head * D + 4 * c;
            *reinterpret_cast<float4 *>(op) = make_float4(o[r][0] * inv, o[r][1] * inv, o[r][2] * inv, o[r][3] * inv);
        } else {
            const int64_t slot = row_index(a, item, head, qi) * a.max_chunks + chunk;
            *reinterpret_cast<float4 *>(a.part_o + slot * D + 4 * c) = make_float4(o[r][0], o[r][1], o[r][2], o[r][3]);
            if (c == 0) *reinterpret_cast<float2 *>(a.part_ml + 2 * slot) = make_float2(m[r], l[r]);
        }
    }
}

// Loads go in batches of ZWG_DECODE_RM_BATCH rows per thread: measured on MI355X, deeper
// per-thread queues stream a cache more slowly, not faster.
// T: keys per tile, 256 or, for short caches, 64 (the planner's split_tile): a chunk then loads
// only the rows it owns, so short caches can be cut into many small chunks that spread over every
// CU instead of a few long ones that leave most CUs idle.
template <int D, int R, int T>
__global__ __launch_bounds__(kDecodeThreads) void decode_rm_kernel(AttnArgs a) {
    constexpr int NT = kDecodeThreads;
    static_assert(T % 64 == 0 && T >= 64, "the softmax pass gives each lane T / 64 keys");
    constexpr int NW = NT / 64;
    constexpr int L = D / 4;   // lanes per key row
    constexpr int P = NT / L;  // key rows per pass
    constexpr int NP = T / P;  // passes over a tile's key rows
#ifndef ZWG_DECODE_RM_BATCH
#define ZWG_DECODE_RM_BATCH 8
#endif
    // loads per thread and batch: 8, or 4 when many rows multiply the operands held with them
    constexpr int MAXB = R > 2 ? 4 : ZWG_DECODE_RM_BATCH;
    constexpr int PB = NP < MAXB ? NP : MAXB; // key/value row loads per batch
    constexpr int RED = NW * R * D;

    __shared__ __align__(16) float q_s[R][D];
    __shared__ __align__(16) float s_s[R][T];
    __shared__ __align__(16) float red[RED];
    __shared__ float alpha_s[R], m_s[R], l_s[R];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    // one workgroup per (item, chunk, KV head), KV head fastest; over the non-empty chunks only
    // when the items have their own key counts (decode_compact_unit; every wave finds the same)
    int hk, chunk, item;
    if (a.n_kv_item && a.n_batch <= kDecodeCompactItems) {
        if (!decode_compact_unit(a, T, blockIdx.x, &item, &chunk, &hk)) return;
    } else {
        hk = blockIdx.x % a.n_head_kv;
        chunk = (blockIdx.x / a.n_head_kv) % a.max_chunks;
        item = blockIdx.x / (a.n_head_kv * a.max_chunks);
    }

    const int n_q = a.n_q;
    const int G = a.group;
    const int rows = n_q * G;
    const int n_kv = item_kv(a, item);
    // the last query sees every key, so the unit's key range is [0, n_kv)
    int chunk_keys;
    const int n_chunks = unit_split(n_kv, T, a.chunk_len, a.max_chunks, &chunk_keys);
    if (chunk >= n_chunks) return;
    const int k_begin = chunk * chunk_keys;
    const int k_end = min(n_kv, k_begin + chunk_keys);
    const int diag = n_kv - n_q;

    const int c = tid % L;     // this thread's 4 dims: 4c .. 4c+3
    const int kslot = tid / L; // this thread's key row within a pass
    // K and V rows through buffer descriptors bounded at the item's last valid row: a row at or
    // past n_kv reads as 0 with no branch (rows in [kn, n_kv) of a split are masked by vlim and
    // get p = 0); per-lane byte offsets sit in VGPRs, per-row ones in SGPRs.
    const uint32_t row_bytes = (uint32_t)a.kv_stride * 4u;
    const uint32_t kv_bytes = n_kv > 0 ? (uint32_t)(n_kv - 1) * row_bytes + 4u * D : 0u;
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(a.k + item * a.k_bstride + (int64_t)hk * D, kv_bytes);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(a.v + item * a.v_bstride + hk * D, kv_bytes);
    const uint32_t lane_off = (uint32_t)kslot * row_bytes + 16u * c;
    // batches of key / value rows held in registers; the first K batch of the first tile is
    // issued before q is staged, the first V batch of a tile before its softmax, and the next
    // tile's first K batch before this tile's P.V, so those latencies overlap other work
    f32x4 kk[PB], vv[PB];
    auto load_k = [&](int k0, int b0) {
#pragma unroll
        for (int i = 0; i < PB; ++i) kk[i] = load_f32x4(krs, lane_off, (uint32_t)(k0 + (b0 + i) * P) * row_bytes);
    };
    auto load_v = [&](int k0, int b0) {
#pragma unroll
        for (int i = 0; i < PB; ++i) vv[i] = load_f32x4(vrs, lane_off, (uint32_t)(k0 + (b0 + i) * P) * row_bytes);
    };
    if (k_begin < k_end) load_k(k_begin, 0);

    // row r = query (r / G) of head hk*G + r % G
    for (int idx = tid; idx < R * D; idx += NT) {
        const int r = idx / D;
        const int p = idx - r * D;
        float val = 0.f;
        if (r < rows) {
            const int qi = r / G;
            const int head = hk * G + (r - qi * G);
            val = load_q(a, item * a.q_bstride + (int64_t)qi * a.q_stride + head * D + p, head * D + p) * a.scale_log2;
        }
        q_s[r][p] = val;
    }
    if (tid < R) {
        m_s[tid] = -INFINITY;
        l_s[tid] = 0.f;
    }
    __syncthreads();

    float qr[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) qr[r][i] = q_s[r][4 * c + i];
    float o[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[r][i] = 0.f;

    for (int k0 = k_begin; k0 < k_end; k0 += T) {
        const int kn = min(T, k_end - k0);
        // ---- scores of this tile into s_s (log2 units)
#pragma unroll 1
        for (int b0 = 0; b0 < NP; b0 += PB) {
            if (b0 > 0) load_k(k0, b0);
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const int j = kslot + (b0 + i) * P;
                float part[R];
#pragma unroll
                for (int r = 0; r < R; ++r)
                    part[r] = qr[r][0] * kk[i][0] + qr[r][1] * kk[i][1] + qr[r][2] * kk[i][2] + qr[r][3] * kk[i][3];
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
        load_v(k0, 0);
        __syncthreads();
        // ---- mask, online softmax; wave w owns rows w, w + NW, ...
        for (int r = wave; r < R; r += NW) {
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
            if (b0 > 0)
                load_v(k0, b0);
            else if (k0 + T < k_end)
                load_k(k0 + T, 0);
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const int j = kslot + (b0 + i) * P;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float p = s_s[r][j];
                    o[r][0] += p * vv[i][0];
                    o[r][1] += p * vv[i][1];
                    o[r][2] += p * vv[i][2];
                    o[r][3] += p * vv[i][3];
                }
            }
        }
        __syncthreads();
    }

    // ---- sum o over the key rows: lanes L apart within a wave, then the NW waves through LDS
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
    for (int idx = tid; idx < R * D; idx += NT) {
        const int r = idx / D;
        const int p = idx - r * D;
        if (r >= rows) continue;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) acc += red[(w * R + r) * D + p];
        const int qi = r / G;
        const int head = hk * G + (r - qi * G);
        if (n_chunks == 1) {
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
    const int64_t blocks = (int64_t)a.max_chunks * a.n_head_kv * a.n_batch;
    if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
    dim3 grid((unsigned)blocks);
    if (grid_blocks) *grid_blocks = (int)blocks;
    const bool kt = a.kt_stride != 0;
    if (kt ? a.split_tile != kDecodeTile : a.split_tile != kDecodeTile && a.split_tile != kDecodeShortTile)
        return hipErrorInvalidValue;
    const int R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : rows <= 6 ? 6 : 8;
    if (rows > kDecodeMaxRows) return hipErrorInvalidValue;
#define ZWG_DEC(DD, RR)                                                                                          \
    if (kt)                                                                                                      \
        decode_kt_kernel<DD, RR><<<grid, dim3(64), 0, stream>>>(a);                                               \
    else if (a.split_tile == kDecodeShortTile)                                                                   \
        decode_rm_kernel<DD, RR, kDecodeShortTile><<<grid, dim3(kDecodeThreads), 0, stream>>>(a);                 \
    else                                                                                                         \
        decode_rm_kernel<DD, RR, kDecodeTile><<<grid, dim3(kDecodeThreads), 0, stream>>>(a);
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
