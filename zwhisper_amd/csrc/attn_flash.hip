// Dense attention on gfx950 fp32 MFMA: one workgroup = 4 waves x 32 query rows of one head,
// streaming 32-key tiles of K and V through LDS, online softmax in registers, the tile loop
// software-pipelined so one tile's softmax overlaps the next tile's score MFMAs.
//
// Replaces the per-(head, 64-row q-block) task of the reference (AttnJob.run,
// src/ops.zig:517-541: S = Q.KT by broadcast FMA, scale, causal limit, softmaxRow, O = S.V)
// without materialising S: each wave keeps its 32x32 score tile in MFMA accumulators.
//
// Layout trick.  The wave computes S^T = K . Q^T with v_mfma_f32_32x32x2_f32 (M = keys,
// N = queries, K = head dims).  Its accumulator register r of lane l holds
// S^T[8*(r/4) + 4*(l/32) + r%4][l%32]: query l%32, a key picked by (r, l/32).  That is exactly
// the B-operand layout of the next product O^T = V^T . P^T (K = keys) if the MFMA at step r
// contracts key 8*(r/4) + 4*(l/32) + r%4 for lane half l/32 -- so the exponentiated scores feed
// the P.V MFMA straight from registers, and only the V^T operand is read in that key order
// (from an LDS tile stored transposed, four consecutive keys per 16-byte read).
// The QK contraction is order-free as well: lane half h contracts dims h*D/2 + s at step s,
// so each lane reads D/2 contiguous floats of its key row and keeps D/2 query values in VGPRs.
//
// Scores are pre-scaled by f32(1/sqrt(d)) * log2(e) (folded into Q) so softmax uses exp2.
#include <type_traits>

#include "attn_kernels.hpp"

namespace zwg {

typedef float f32x16 __attribute__((ext_vector_type(16)));

static __device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

#ifndef ZWG_SCHED_INTERLEAVE
#define ZWG_SCHED_INTERLEAVE 0
#endif
#ifndef ZWG_RESCALE_SLACK
#define ZWG_RESCALE_SLACK 8.0f
#endif

template <int D, bool KT>
__global__ __launch_bounds__(256) void flash_attn_kernel(AttnArgs a) {
    constexpr int BM = kFlashBM;
    constexpr int BN = kFlashBN;
    constexpr int HD = D / 2;   // dims per lane half in the QK contraction
    constexpr int KS = D + 4;   // LDS row stride of the K tile [key][dim]
    constexpr int VS = BN + 4;  // LDS row stride of the V^T tile [dim][key]
    constexpr int NDB = D / 32; // 32-dim output tiles
    constexpr int LD = BN * D / 4 / 256; // float4 loads per thread per tile, per tensor
    static_assert(LD >= 1, "tile too small for the workgroup");

    __shared__ __align__(16) float Ks[2][BN * KS];
    __shared__ __align__(16) float Vt[2][D * VS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int n_qblocks = (a.n_q + BM - 1) / BM;
    int chunk, qb, ih;
    dense_unit(a, n_qblocks, BM, BN, &qb, &chunk, &ih);
    const int item = ih / a.n_head;
    const int head = ih - item * a.n_head;
    const int hk = head / a.group;

    const int n_q = a.n_q;
    const int n_kv = item_kv(a, item);
    const int q_first = qb * BM;
    const int q_end_blk = min(q_first + BM, n_q);
    const int kv_hi = a.causal ? max(0, n_kv - n_q + q_end_blk) : n_kv;
    int chunk_keys;
    const int n_chunks = unit_split(kv_hi, BN, a.chunk_len, a.max_chunks, &chunk_keys);
    if (chunk >= n_chunks) return;
    const int k_begin = chunk * chunk_keys;
    const int k_end = min(kv_hi, k_begin + chunk_keys);

    const float *qp = a.q + item * a.q_bstride + head * D;
    const float *kp = a.k + item * a.k_bstride + (KT ? (int64_t)hk * D * a.kt_stride : (int64_t)hk * D);
    const float *vp = a.v + item * a.v_bstride + hk * D;

    // This lane's query row and the wave's key window.
    const int q_wave = q_first + wave * 32;
    const int query = q_wave + col;
    const bool q_valid = query < n_q;
    const bool wave_active = q_wave < n_q;
    const int q_wave_last = min(q_wave + 31, n_q - 1);
    const int diag = n_kv - n_q; // query i sees keys j <= diag + i
    // keys the wave needs at all (exclusive), and keys every query of the wave sees
    const int wave_hi = min(k_end, a.causal ? diag + q_wave_last + 1 : n_kv);
    const int wave_full = min(k_end, a.causal ? diag + q_wave + 1 : n_kv);

    // this lane's query, pre-scaled into log2 units (loaded after the first tile's K and V loads
    // are issued, so the three wait out one memory latency)
    float qreg[HD];

    f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (f32x16){0};
    float m_run = -INFINITY;
    float l_run = 0.f;

    // Tile staging.  K runs two tiles ahead of the tile being finished and V one tile ahead,
    // so that in iteration t the MFMAs of S(t+1) (from K(t+1)) can overlap the softmax of
    // tile t, and the LDS buffers read in an iteration (K(t+1), V(t)) are never the ones
    // written in it (K(t+2), V(t+1)): one barrier per tile suffices.  Each thread holds what it
    // stores as 16-byte quads: four dims of one key for K (row-major K: one 16-byte load;
    // transposed K: four coalesced dword loads, one per dim row) and four keys of one dim for V^T
    // (four coalesced dword loads, one per key row), each stored with one 16-byte LDS write.
    // Loads go through buffer descriptors (no branches, offsets as a per-lane base plus a
    // wave-uniform part): V and row-major K end at the item's last key row, so a key at or past
    // n_kv reads 0; transposed K ends at the last dim row's n_kv-th column, and a key past n_kv
    // in an earlier dim row reads that row's padding (finite by the reference's contract,
    // src/ops.zig:477-492) -- masked out of the scores either way.
    constexpr int NG = D / 32;    // quads per thread per tile, per tensor
    constexpr int VTPD = 256 / D; // V: threads per dim
    static_assert(NG == LD, "each thread stages D/32 quads of each tile");
    f32x4 kr[NG], vr[NG];
    const int k_key = tid % BN, k_dq = tid / BN;   // transposed K: key, first dim quad
    const int v_dim = tid % D, v_kq = tid / D;     // V: dim, first key quad
    auto k_dim = [&](int g) { return 4 * (k_dq + 8 * g); };   // transposed K: quads k_dq, k_dq + 8, ..
    auto v_key = [&](int g) { return 4 * (v_kq + VTPD * g); }; // V: quads v_kq, v_kq + VTPD, ..
    const uint32_t row_b = (uint32_t)a.kv_stride * 4u;
    const uint32_t kv_span = n_kv > 0 ? (uint32_t)(n_kv - 1) * row_b + 4u * D : 0u;
    const uint32_t kt_span = n_kv > 0 ? (uint32_t)((D - 1) * a.kt_stride + n_kv) * 4u : 0u;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(kp), 0, (int)(KT ? kt_span : kv_span), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(vp), 0, (int)kv_span, 0x00020000);
    const uint32_t kt_row_b = (uint32_t)a.kt_stride * 4u;
    const uint32_t k_base = KT ? (uint32_t)k_dim(0) * kt_row_b + 4u * (uint32_t)k_key
                               : (uint32_t)(tid / (D / 4)) * row_b + 16u * (uint32_t)(tid % (D / 4));
    const uint32_t v_base = (uint32_t)v_key(0) * row_b + 4u * (uint32_t)v_dim;
    auto load_k_to = [&](f32x4 (&dst)[NG], int k0) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (KT) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    dst[g][j] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(
                                   krs, (int)k_base, (int)((uint32_t)k0 * 4u + (uint32_t)(32 * g + j) * kt_row_b), 0));
            } else {
                dst[g] = __builtin_bit_cast(
                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               krs, (int)k_base, (int)((uint32_t)(k0 + (1024 / D) * g) * row_b), 0));
            }
        }
    };
    auto load_k = [&](int k0) { load_k_to(kr, k0); };
    auto load_v = [&](int k0) {
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                vr[g][j] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(
                               vrs, (int)v_base, (int)((uint32_t)(k0 + 4 * VTPD * g + j) * row_b), 0));
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            int key, dim;
            if (KT) {
                key = k_key;
                dim = k_dim(g);
            } else {
                const int f = tid + 256 * g;
                key = f / (D / 4);
                dim = 4 * (f % (D / 4));
            }
            *reinterpret_cast<f32x4 *>(&Ks[buf][key * KS + dim]) = kr[g];
        }
    };
    auto store_v = [&](int buf) {
#pragma unroll
        for (int g = 0; g < NG; ++g) *reinterpret_cast<f32x4 *>(&Vt[buf][v_dim * VS + v_key(g)]) = vr[g];
    };
    // S^T tile = K . Q^T (32 keys x 32 queries) from the K buffer
    auto qk = [&](int buf) {
        f32x16 sc = (f32x16){0};
        const float *krow = &Ks[buf][col * KS + half * HD];
#pragma unroll
        for (int j = 0; j < HD; j += 4) {
            const f32x4 kk = *reinterpret_cast<const f32x4 *>(krow + j);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[0], qreg[j + 0], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[1], qreg[j + 1], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[2], qreg[j + 2], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[3], qreg[j + 3], sc, 0, 0, 0);
        }
        return sc;
    };
    // mask keys past the chunk end or past this query's causal limit, then move the running
    // max.  It only moves when a tile's max exceeds it by more than ZWG_RESCALE_SLACK (log2
    // units): until then p = 2^(s - m_run) stays below 2^slack while o and l keep sharing one
    // reference point, so the final o / l is unchanged and the rescale of o runs on the first
    // tile and almost never after.  The lane holds 16 of its query's 32 keys, the partner lane
    // (l ^ 32) the other 16.
    auto mask_and_max = [&](f32x16 &sc, int k0) {
        if (k0 + BN > wave_full) {
            const int lim = min(k_end, a.causal ? diag + query + 1 : n_kv);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r >> 2) + 4 * half + (r & 3);
                sc[r] = key < lim ? sc[r] : -INFINITY;
            }
        }
        float mt = sc[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mt = fmaxf(mt, sc[r]);
        mt = lane_pair_max(mt);
        if (__any(mt > m_run + ZWG_RESCALE_SLACK)) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = m_run == -INFINITY ? 0.f : exp2_fast(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db] *= alpha;
            m_run = m_new;
        }
    };
    auto exp_sum = [&](f32x16 &sc) {
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = exp2_fast(sc[r] - m_use);
            ls += sc[r];
        }
        l_run += ls;
    };
    // qk() of the next tile fused with exp_sum() of this one, in a fixed issue order: after
    // each score MFMA comes one step of the exponentials, so the VALU work executes while the
    // MFMA pipe is busy with the (dependent) MFMA chain.  The K operand is read one group ahead.
    auto qk_exp = [&](int buf, f32x16 &p) {
        constexpr int EVERY = HD / 16; // MFMA steps per exponential
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float ls = 0.f;
        f32x16 sc = (f32x16){0};
        const float *krow = &Ks[buf][col * KS + half * HD];
        f32x4 kk = *reinterpret_cast<const f32x4 *>(krow);
#pragma unroll
        for (int j = 0; j < HD; j += 4) {
            const f32x4 kn = j + 4 < HD ? *reinterpret_cast<const f32x4 *>(krow + j + 4) : kk;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[u], qreg[j + u], sc, 0, 0, 0);
                if ((j + u) % EVERY == 0) {
                    const int r = (j + u) / EVERY;
                    p[r] = exp2_fast(p[r] - m_use);
                    ls += p[r];
                }
#if ZWG_SCHED_INTERLEAVE
                __builtin_amdgcn_sched_barrier(0);
#endif
            }
            kk = kn;
        }
        l_run += ls;
        return sc;
    };
    // O^T += V^T . P^T from the V buffer
    auto pv = [&](const f32x16 &p, int buf) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const float *vrow = &Vt[buf][(db * 32 + col) * VS + 4 * half];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 vv = *reinterpret_cast<const f32x4 *>(vrow + 8 * g);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[0], p[4 * g + 0], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[1], p[4 * g + 1], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[2], p[4 * g + 2], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[3], p[4 * g + 3], o[db], 0, 0, 0);
            }
        }
    };
    auto wave_needs = [&](int k0) { return wave_active && k0 < wave_hi; };

    const int n_tiles = k_end > k_begin ? (k_end - k_begin + BN - 1) / BN : 0;
    f32x16 s_cur = (f32x16){0};
    // tile 1's K goes out with tile 0's K and V and the queries: the prologue waits out one memory
    // round trip, not two
    f32x4 kr1[NG];
    if (n_tiles > 0) {
        load_k(k_begin);
        load_v(k_begin);
    }
    if (n_tiles > 1) load_k_to(kr1, k_begin + BN);
    if (q_valid) {
        const f32x4 *src = reinterpret_cast<const f32x4 *>(qp + (int64_t)query * a.q_stride + half * HD);
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) {
            const f32x4 t = src[i];
            qreg[4 * i + 0] = t[0] * a.scale_log2;
            qreg[4 * i + 1] = t[1] * a.scale_log2;
            qreg[4 * i + 2] = t[2] * a.scale_log2;
            qreg[4 * i + 3] = t[3] * a.scale_log2;
        }
    } else {
#pragma unroll
        for (int i = 0; i < HD; ++i) qreg[i] = 0.f;
    }
    if (n_tiles > 0) {
        store_k(0);
        store_v(0);
        if (n_tiles > 1)
#pragma unroll
            for (int g = 0; g < NG; ++g) kr[g] = kr1[g];
    }
    __syncthreads();
    if (n_tiles > 0 && wave_needs(k_begin)) s_cur = qk(0);
    if (n_tiles > 1) store_k(1);
    __syncthreads();

    // one tile: t's buffer parity is a compile-time constant (the loop runs two tiles per turn),
    // so LDS addresses are immediate offsets and the score registers alternate between s_cur and
    // s_b without copies
    auto step = [&](auto parity, int t, f32x16 &s_this, f32x16 &s_next) {
        constexpr int cur = decltype(parity)::value, nxt = cur ^ 1;
        const int k0 = k_begin + t * BN;
        if (t + 2 < n_tiles) load_k(k0 + 2 * BN);
        if (t + 1 < n_tiles) load_v(k0 + BN);
        const bool need_cur = wave_needs(k0);
        const bool need_next = t + 1 < n_tiles && wave_needs(k0 + BN);
        if (need_cur) mask_and_max(s_this, k0);
        if (need_cur && need_next) {
            // the MFMAs of the next tile's scores and this tile's exponentials are independent:
            // issued in one block, the VALU work runs while the MFMA pipe is busy
            s_next = qk_exp(nxt, s_this);
        } else if (need_cur) {
            exp_sum(s_this);
        } else if (need_next) {
            s_next = qk(nxt);
        }
        if (need_cur) pv(s_this, cur);
        if (t + 2 < n_tiles) store_k(cur);
        if (t + 1 < n_tiles) store_v(nxt);
        __syncthreads();
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    f32x16 s_b = (f32x16){0};
    int t = 0;
    for (; t + 1 < n_tiles; t += 2) {
        step(P0{}, t, s_cur, s_b);
        step(P1{}, t + 1, s_b, s_cur);
    }
    if (t < n_tiles) step(P0{}, t, s_cur, s_b);

    const float l_tot = lane_pair_sum(l_run);
    // lane holds dims db*32 + 8*g + 4*half + {0..3} in registers 4g..4g+3 of o[db]
    if (n_chunks == 1) { // an unsplit unit writes its rows itself; the merge pass skips them
        uint32_t big = 0;
        if (q_valid) {
            const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
            float *op = a.out + item * a.out_bstride + (int64_t)query * a.out_stride + head * D;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4 w = {o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv};
                    *reinterpret_cast<f32x4 *>(op + db * 32 + 8 * g + 4 * half) = w;
                    big = max(max(big, max(abs_bits(w[0]), abs_bits(w[1]))), max(abs_bits(w[2]), abs_bits(w[3])));
                }
        }
        if (a.out_max) out_max_record(a, big); // every lane of the wave takes part
        return;
    }
    if (!q_valid) return;
    const int64_t slot = row_index(a, item, head, query) * a.max_chunks + chunk;
    float *po = a.part_o + slot * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 w = {o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
            *reinterpret_cast<f32x4 *>(po + db * 32 + 8 * g + 4 * half) = w;
        }
    if (half == 0) {
        a.part_ml[2 * slot] = m_run;
        a.part_ml[2 * slot + 1] = l_tot;
    }
}

// Merge the split-KV partials of each row:
//   out = sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c,   M = max_c m_c,
// one thread per (row, 4 dims).  MAXC > 0: the call has at most MAXC splits per row.
template <int D, int MAXC>
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs a) {
    // the merge of one (row, 4 dims); returns the largest |value| written as its bit pattern, or 0
    auto merge = [&]() -> uint32_t {
        constexpr int G4 = D / 4;
        const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
        const int64_t n_rows = (int64_t)a.n_batch * a.n_head * a.n_q;
        const int64_t row = t / G4;
        if (row >= n_rows) return 0u;
        const int g = (int)(t - row * G4);
        const int query = (int)(row % a.n_q);
        const int64_t ih = row / a.n_q;
        const int head = (int)(ih % a.n_head);
        const int item = (int)(ih / a.n_head);
        const float2 *ml = reinterpret_cast<const float2 *>(a.part_ml) + row * a.max_chunks;
        const float4 *po = reinterpret_cast<const float4 *>(a.part_o + row * a.max_chunks * D) + g;
        const int q_end = min((query / a.rows_per_unit + 1) * a.rows_per_unit, a.n_q);
        auto row_chunks = [&](int n_kv) {
            const int kv_hi = a.causal ? max(0, n_kv - a.n_q + q_end) : n_kv;
            int chunk_keys;
            return unit_split(kv_hi, a.split_tile, a.chunk_len, a.max_chunks, &chunk_keys);
        };
        // With one key count for every item the row's chunk count is known at once: rows the
        // attention kernel finished (one chunk) load nothing, and the others load their own slots
        // only.  With per-item counts in device memory, every slot of the row (c < max_chunks, all
        // inside the workspace) is loaded before the count arrives, so the partials' round trip
        // overlaps that of the count; slots past the row's chunk count are discarded below by
        // selection (they may hold anything).
        const int known_chunks = a.n_kv_item ? 0 : row_chunks(a.n_kv);
        if (known_chunks == 1) return 0u; // written by the attention kernel
        const int last_slot = (known_chunks ? known_chunks : a.max_chunks) - 1;
        float2 mlr[MAXC > 0 ? MAXC : 1];
        float4 vr[MAXC > 0 ? MAXC : 1];
        if (MAXC > 0) {
#pragma unroll
            for (int c = 0; c < MAXC; ++c) { // slots past the last reload it: no branches
                const int cc = min(c, last_slot);
                mlr[c] = ml[cc];
                vr[c] = po[(int64_t)cc * G4];
            }
        }
        const int n_chunks = known_chunks ? known_chunks : row_chunks(item_kv(a, item));
        if (n_chunks == 1) return 0u; // written by the attention kernel

        float M = -INFINITY, L = 0.f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        if (MAXC > 0) {
            // merged from registers: the row's first n_chunks slots only
#pragma unroll
            for (int c = 0; c < MAXC; ++c)
                if (c < n_chunks) M = fmaxf(M, mlr[c].x);
            if (M != -INFINITY) {
#pragma unroll
                for (int c = 0; c < MAXC; ++c) {
                    if (c >= n_chunks) continue;
                    const float w = exp2_fast(mlr[c].x - M); // 0 for a split that saw no key of this row
                    L += w * mlr[c].y;
                    acc.x += w * vr[c].x;
                    acc.y += w * vr[c].y;
                    acc.z += w * vr[c].z;
                    acc.w += w * vr[c].w;
                }
            }
        } else {
            // two passes whose loads do not depend on each other, so they are all in flight at once
#pragma unroll 8
            for (int c = 0; c < n_chunks; ++c) M = fmaxf(M, ml[c].x);
            if (M != -INFINITY) {
#pragma unroll 8
                for (int c = 0; c < n_chunks; ++c) {
                    const float2 m_l = ml[c];
                    const float4 v = po[(int64_t)c * G4];
                    const float w = exp2_fast(m_l.x - M);
                    L += w * m_l.y;
                    acc.x += w * v.x;
                    acc.y += w * v.y;
                    acc.z += w * v.z;
                    acc.w += w * v.w;
                }
            }
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        float *op = a.out + item * a.out_bstride + (int64_t)query * a.out_stride + head * D + 4 * g;
        const float4 w = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        *reinterpret_cast<float4 *>(op) = w;
        return max(max(abs_bits(w.x), abs_bits(w.y)), max(abs_bits(w.z), abs_bits(w.w)));
    };
    const uint32_t big = merge();
    if (a.out_max) out_max_record(a, big); // every lane of the wave takes part

}

hipError_t launch_flash(const AttnArgs &a, int d, hipStream_t stream, int *grid_blocks) {
    const int n_qblocks = (a.n_q + kFlashBM - 1) / kFlashBM;
    const int max_chunks = a.max_chunks;
    const int64_t blocks = a.heavy_first == 2 ? a.live_blocks : (int64_t)max_chunks * n_qblocks * a.n_batch * a.n_head;
    if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
    dim3 grid((unsigned)blocks);
    dim3 block(256);
    if (grid_blocks) *grid_blocks = (int)(grid.x * grid.y * grid.z);
    const bool kt = a.kt_stride != 0;
#define ZWG_FLASH(DD)                                                                                            \
    if (kt)                                                                                                      \
        flash_attn_kernel<DD, true><<<grid, block, 0, stream>>>(a);                                              \
    else                                                                                                         \
        flash_attn_kernel<DD, false><<<grid, block, 0, stream>>>(a);
    switch (d) {
    case 32: ZWG_FLASH(32) break;
    case 64: ZWG_FLASH(64) break;
    case 128: ZWG_FLASH(128) break;
    default: return hipErrorInvalidValue;
    }
#undef ZWG_FLASH
    return hipGetLastError();
}

hipError_t launch_combine(const AttnArgs &a, int d, hipStream_t stream) {
    const int64_t n_rows = (int64_t)a.n_batch * a.n_head * a.n_q;
    // A small merge (decode: one row per item and head) as 64-thread workgroups, so its single
    // round of loads comes from every CU rather than a few: the Qwen decode step 1.1 us faster,
    // the small.en step 0.9 us, tiny.en 0.5 us.  Merges of 1024 or more 256-thread workgroups
    // (the prefill) stay at 256, which measured 0.4 us faster there.
    const int64_t threads = n_rows * (d / 4);
    const int bs = threads < 1024ll * 256 ? 64 : 256;
    dim3 grid((unsigned)((threads + bs - 1) / bs));
    dim3 block(bs);
#define ZWG_COMBINE(DD)                                                                                          \
    if (a.max_chunks <= 4)                                                                                       \
        combine_kernel<DD, 4><<<grid, block, 0, stream>>>(a);                                                    \
    else if (a.max_chunks <= 16)                                                                                 \
        combine_kernel<DD, 16><<<grid, block, 0, stream>>>(a);                                                   \
    else                                                                                                         \
        combine_kernel<DD, 0><<<grid, block, 0, stream>>>(a);
    switch (d) {
    case 32: ZWG_COMBINE(32) break;
    case 64: ZWG_COMBINE(64) break;
    case 128: ZWG_COMBINE(128) break;
    default: return hipErrorInvalidValue;
    }
#undef ZWG_COMBINE
    return hipGetLastError();
}

} // namespace zwg
