// Dense attention on gfx950 f16 MFMA with f32-level accuracy: the fp32 kernel of attn_flash.hip
// (same workgroup geometry, tile pipeline, online softmax, split and merge), with each product of
// Q.K^T and P.V computed as three f16 MFMA products of split operands.
//
// Split.  Every f32 operand x is written as hi + lo with hi = f16(x), lo = f16(x - hi) (together
// 22 significand bits), and a product a.b as ah.bh + ah.bl + al.bh (al.bl is below the rounding of
// lo), each on a 32x32x16 MFMA with f32 accumulation: 12 MFMAs per 32 x 32 tile of Q.K^T (d = 64)
// and 12 for P.V, against 64 fp32 MFMAs of 32x32x2, so about 5x fewer MFMA cycles.
//   A score's error is absolute in the exponent, so it must not grow with the scores: with bf16
//   terms (16 bits) it does, by 2^-17 of sum |q_i k_i|, and scores spread 16x wider than
//   unit-variance inputs give (large-logit heads) already cost 3e-4 at the output; with f16 the
//   same inputs stay near 2e-5 (CPU emulation against f64).  P.V on f16 terms keeps the output's
//   error near 2^-23 of |V| (bf16 terms gave 2^-17: measured 2e-5 on the Qwen2 prefill, 8e-7 now).
//   f16's range is the price: Q enters pre-scaled by log2(e)/sqrt(d), and K and V must stay
//   below 65504 in magnitude.  A larger key gives an infinite hi term and NaN in the rows that see
//   it (a masked key is replaced by -inf before the softmax and cannot poison anything); a larger
//   value gives NaN in its own output column of every row whose wave loads its 32-key tile, since
//   inf - inf and 0 * inf are NaN -- never a silently wrong finite result.  P is at most 2^8 by the lazily moved running max.  f16 subnormals are
//   kept by the MFMA, so small lo terms keep their absolute accuracy.
//
// Operands.  S^T = K . Q^T (M = keys, N = queries, K = head dims): lane l of the A operand (K)
// holds key l%32, dims 16 j + 8 (l/32) + 0..7 of k-step j; the B operand (Q^T) the same dims of
// query l%32, split once into registers.  The result layout of every 32x32 MFMA is the one the
// fp32 kernel uses (register r of lane l: key 8 (r/4) + 4 (l/32) + r%4 of query l%32), so the
// masking and softmax are unchanged.  For O^T = V^T . P^T, k-step s contracts the keys of
// registers 8 s .. 8 s + 7, which for lane half h are keys 16 s + 4 h + 0..3 and 16 s + 8 + 4 h
// + 0..3: the V^T tile is stored with keys 4..7 and 8..11 of every 16 swapped, so each lane's
// eight keys are contiguous and one 16-byte read.
//
// LDS.  K tiles [key][dim] and V^T tiles [dim][key], f16 hi and lo planes, double-buffered,
// 16-byte chunks XOR-swizzled by row so a wave's operand reads are conflict-free.
#include <type_traits>

#include "attn_kernels.hpp"
#include "kv_image.hpp"

namespace zwg {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

typedef float f32x8 __attribute__((ext_vector_type(8)));

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// f16 split of a pair, four VALU: one v_cvt_pk_f16_f32 rounds the pair; v_fma_mix_f32 reads each
// half as f16 and forms x - hi in f32 in one instruction (exact: hi is x rounded, so x - hi is
// representable); a second v_cvt_pk rounds the remainders.
__device__ __forceinline__ float sub_f16_lo(uint32_t pair, float x) { // x - (float)low half of pair
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(x));
    return r;
}
__device__ __forceinline__ float sub_f16_hi(uint32_t pair, float x) { // x - (float)high half of pair
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(x));
    return r;
}
__device__ __forceinline__ uint32_t split2_f16(float a, float b, uint32_t &lo) {
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){sub_f16_lo(h, a), sub_f16_hi(h, b)}, f16x2));
    return h;
}
__device__ __forceinline__ void split8(const f32x8 &x, f16x8 &hi, f16x8 &lo) {
    u32x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t li;
        h[i] = split2_f16(x[2 * i], x[2 * i + 1], li);
        l[i] = li;
    }
    hi = __builtin_bit_cast(f16x8, h);
    lo = __builtin_bit_cast(f16x8, l);
}
__device__ __forceinline__ void split4(const f32x4 &x, f16x4 &hi, f16x4 &lo) {
    u32x2 h, l;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t li;
        h[i] = split2_f16(x[2 * i], x[2 * i + 1], li);
        l[i] = li;
    }
    hi = __builtin_bit_cast(f16x4, h);
    lo = __builtin_bit_cast(f16x4, l);
}

// LDS tile layouts (kv_image.hpp): K [key][dim] and V^T [dim][key position], XOR-swizzled
template <int D>
__device__ __forceinline__ int k_at(int key, int dim) { return zwg_img::k_at<D>(key, dim); }
__device__ __forceinline__ int v_pos(int key) { return zwg_img::v_pos(key); }
__device__ __forceinline__ int v_at(int dim, int pos) { return zwg_img::v_at(dim, pos); }

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt 6:4 and lgkmcnt 11:8 left at their maxima)
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

} // namespace

// d = 128 needs just over 256 VGPRs unconstrained; capping it there keeps two waves per SIMD.
// PL: K and V come as tile images (kv_image.hpp: a.k_img, a.v_img), copied into LDS by the
// buffer loads' LDS mode with no registers and no split; a.k and a.v are not read.
// (PL at d = 64 needs 145 VGPRs, three waves per SIMD; capped at 128 for a fourth it spills and
// measured no faster.)
template <int D, bool KT, bool PL = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 ? 2 : 1)))
void flash_x3_kernel(AttnArgs a) {
    static_assert(!PL || (!KT && D >= 64), "tile images: row-major K, whole 4 KB planes");
    constexpr int BM = kFlashBM;
    constexpr int BN = kFlashBN;
    constexpr int NKS = D / 16;  // k-steps of the QK product
    constexpr int NDB = D / 32;  // 32-dim output tiles
    static_assert(BN * D == 256 * 4 * (D / 32), "each thread stages D/32 quads of each tile");
    static_assert(BN == 32, "the P.V key order assumes 32-key tiles");

    __shared__ __align__(16) _Float16 Kh[2][BN * D];
    __shared__ __align__(16) _Float16 Kl[2][BN * D];
    __shared__ __align__(16) _Float16 Vh[2][D * BN];
    __shared__ __align__(16) _Float16 Vl[2][D * BN];

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

    const int q_wave = q_first + wave * 32;
    const int query = q_wave + col;
    const bool q_valid = query < n_q;
    const bool wave_active = q_wave < n_q;
    const int q_wave_last = min(q_wave + 31, n_q - 1);
    const int diag = n_kv - n_q; // query i sees keys j <= diag + i
    const int wave_hi = min(k_end, a.causal ? diag + q_wave_last + 1 : n_kv);
    const int wave_full = min(k_end, a.causal ? diag + q_wave + 1 : n_kv);

    // this lane's query, pre-scaled into log2 units, dims 16 j + 8 half + 0..7, split (loaded
    // after the first tile's K and V loads are issued, so the two wait out one memory latency)
    f16x8 qh[NKS], ql[NKS];

    f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (f32x16){0};
    float m_run = -INFINITY;
    float l_run = 0.f;

    // Tile staging as in flash_attn_kernel: K two tiles ahead, V one tile ahead, one barrier per
    // tile.  Each thread holds what it stores as contiguous 16-bit quads: four dims of one key for K
    // (row-major K: one 16-byte load; transposed K: four coalesced dword loads, one per dim row)
    // and four keys of one dim for V^T (four coalesced dword loads, one per key row).
    constexpr int NG = D / 32;        // quads per thread per tile, per tensor
    constexpr int VTPD = 256 / D;     // V: threads per dim
    f32x4 kr[NG], vr[NG];
    const int k_key = tid % BN, k_dq = tid / BN;   // transposed K: key, first dim quad
    const int v_dim = tid % D, v_kq = tid / D;     // V: dim, first key quad
    auto k_dim = [&](int g) { return 4 * (k_dq + 8 * g); };   // transposed K: quads k_dq, k_dq + 8, ..
    auto v_key = [&](int g) { return 4 * (v_kq + VTPD * g); }; // V: quads v_kq, v_kq + VTPD, ..
    // Branch-free loads through buffer descriptors (32-bit byte offsets; the host keeps an item's
    // K and V spans below 2 GiB): V and row-major K end at the item's last key row, so a key at or
    // past n_kv reads 0; transposed K ends at the last dim row's n_kv-th column, and a key past
    // n_kv in an earlier dim row reads that row's padding (finite by the reference's contract,
    // src/ops.zig:477-492) -- masked out of the scores either way.  Each offset is a per-lane base
    // fixed for the whole loop (one VGPR per tensor) plus a wave-uniform part in an SGPR: the
    // tile's first key and the step between a thread's quads and elements.
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
    // PL: this (item, KV head)'s images; wave w copies bytes [1024 w, 1024 w + 1024) of every 4 KB
    // piece of a tile's planes, lane l 16 of them
    constexpr int PIECES = 32 * D * 2 / 4096; // 4 KB pieces of one plane
    constexpr int IMG_LOADS = 2 * PIECES;     // copies per wave per tile of K (or of V)
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const int64_t img_ih = (int64_t)item * a.n_head_kv + hk;
    const uint32_t img_bytes = PL ? (uint32_t)a.img_tiles * (uint32_t)zwg_img::block_halves(D) * 2u : 0u;
    const __amdgpu_buffer_rsrc_t kimg = __builtin_amdgcn_make_buffer_rsrc(
        PL ? const_cast<_Float16 *>(a.k_img + zwg_img::block_offset(img_ih, a.img_tiles, 0, D)) : nullptr, 0,
        (int)img_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vimg = __builtin_amdgcn_make_buffer_rsrc(
        PL ? const_cast<_Float16 *>(a.v_img + zwg_img::block_offset(img_ih, a.img_tiles, 0, D)) : nullptr, 0,
        (int)img_bytes, 0x00020000);
    auto copy_tile = [&](__amdgpu_buffer_rsrc_t src, int k0, _Float16 *hi_dst, _Float16 *lo_dst) {
        const uint32_t t_off = (uint32_t)(k0 / BN) * (uint32_t)zwg_img::block_halves(D) * 2u;
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
#pragma unroll
            for (int c = 0; c < PIECES; ++c) {
                const int in_plane = c * 4096 + wave_u * 1024; // bytes
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    src, (__attribute__((address_space(3))) void *)((pl ? lo_dst : hi_dst) + in_plane / 2), 16,
                    (int)(t_off + (uint32_t)(pl * 32 * D * 2 + in_plane) + 16u * (uint32_t)lane), 0, 0, 0);
            }
    };
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
            f16x4 h, l;
            split4(kr[g], h, l);
            *reinterpret_cast<f16x4 *>(&Kh[buf][k_at<D>(key, dim)]) = h;
            *reinterpret_cast<f16x4 *>(&Kl[buf][k_at<D>(key, dim)]) = l;
        }
    };
    auto store_v = [&](int buf) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            f16x4 h, l;
            split4(vr[g], h, l);
            const int at = v_at(v_dim, v_pos(v_key(g))); // keys 4q .. 4q+3 sit at four consecutive positions
            *reinterpret_cast<f16x4 *>(&Vh[buf][at]) = h;
            *reinterpret_cast<f16x4 *>(&Vl[buf][at]) = l;
        }
    };
    // one k-step of S^T = K . Q^T: three f16 products
    auto qk_step = [&](int buf, int j, f32x16 sc) {
        const int at = k_at<D>(col, 16 * j + 8 * half);
        const f16x8 kh = *reinterpret_cast<const f16x8 *>(&Kh[buf][at]);
        const f16x8 kl = *reinterpret_cast<const f16x8 *>(&Kl[buf][at]);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[j], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, ql[j], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, qh[j], sc, 0, 0, 0);
        return sc;
    };
    auto qk = [&](int buf) {
        f32x16 sc = (f32x16){0};
#pragma unroll
        for (int j = 0; j < NKS; ++j) sc = qk_step(buf, j, sc);
        return sc;
    };
    // masking and the lazily moved running max, as flash_attn_kernel
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
        if (__any(mt > m_run + 8.0f)) {
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
        float ls;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = exp2_fast(sc[r] - m_use);
            ls = r == 0 ? sc[0] : ls + sc[r];
        }
        l_run += ls;
    };
    // the next tile's score MFMAs interleaved with this tile's exponentials
    auto qk_exp = [&](int buf, f32x16 &p) {
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float ls;
        f32x16 sc = (f32x16){0};
        constexpr int PER = 16 / NKS; // exponentials per k-step
#pragma unroll
        for (int j = 0; j < NKS; ++j) {
            sc = qk_step(buf, j, sc);
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int r = j * PER + u;
                p[r] = exp2_fast(p[r] - m_use);
                ls = r == 0 ? p[0] : ls + p[r];
            }
        }
        l_run += ls;
        return sc;
    };
    // O^T += V^T . P^T: k-step s contracts registers 8 s .. 8 s + 7 of p.  The block runs at raised
    // wave priority, so a wave that reaches its MFMA chain issues ahead of the waves in their
    // exponentials and keeps the matrix pipe fed (base.en 1-2% faster; priority 3 measured the
    // same, and raising it around the MFMAs alone, without the P split, slower)
    auto pv = [&](const f32x16 &p, int buf) {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            f32x8 pr;
#pragma unroll
            for (int e = 0; e < 8; ++e) pr[e] = p[8 * s + e];
            f16x8 ph, pl;
            split8(pr, ph, pl);
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const int at = v_at(db * 32 + col, 16 * s + 8 * half);
                const f16x8 vh = *reinterpret_cast<const f16x8 *>(&Vh[buf][at]);
                const f16x8 vl = *reinterpret_cast<const f16x8 *>(&Vl[buf][at]);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, ph, o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pl, o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, ph, o[db], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
    };
    auto wave_needs = [&](int k0) { return wave_active && k0 < wave_hi; };

    const int n_tiles = k_end > k_begin ? (k_end - k_begin + BN - 1) / BN : 0;
    f32x16 s_cur = (f32x16){0};
    // tile 1's K goes out with tile 0's K and V and the queries, so the prologue waits out one
    // memory round trip, not two (the loop then keeps its one-tile-ahead staging)
    f32x4 kr1[NG];
    if constexpr (PL) {
        if (n_tiles > 0) {
            copy_tile(vimg, k_begin, Vh[0], Vl[0]);
            copy_tile(kimg, k_begin, Kh[0], Kl[0]);
        }
        if (n_tiles > 1) copy_tile(kimg, k_begin + BN, Kh[1], Kl[1]);
    } else {
        if (n_tiles > 0) {
            load_k(k_begin);
            load_v(k_begin);
        }
        if (n_tiles > 1) load_k_to(kr1, k_begin + BN);
    }
    {
        // all of the row's loads go out together, then one wait
        f32x4 qraw[2 * NKS];
        if (q_valid) {
            const f32x4 *src = reinterpret_cast<const f32x4 *>(qp + (int64_t)query * a.q_stride + 8 * half);
#pragma unroll
            for (int j = 0; j < NKS; ++j) {
                qraw[2 * j] = src[4 * j];
                qraw[2 * j + 1] = src[4 * j + 1];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2 * NKS; ++j) qraw[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < NKS; ++j) {
            f32x8 qv;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qv[e] = qraw[2 * j][e] * a.scale_log2;
                qv[4 + e] = qraw[2 * j + 1][e] * a.scale_log2;
            }
            split8(qv, qh[j], ql[j]);
        }
    }
    if constexpr (PL) {
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    } else if (n_tiles > 0) {
        store_k(0);
        store_v(0);
        if (n_tiles > 1)
#pragma unroll
            for (int g = 0; g < NG; ++g) kr[g] = kr1[g];
    }
    __syncthreads();
    if (n_tiles > 0 && wave_needs(k_begin)) s_cur = qk(0);
    if (!PL && n_tiles > 1) store_k(1);
    __syncthreads(); // PL: every wave is done with tile 0's K before tile 2 is copied over it

    // one tile: t's buffer parity is a compile-time constant (the loop runs two tiles per turn),
    // so LDS addresses are immediate offsets and the score registers alternate between sa and sb
    // without copies
    auto step = [&](auto parity, int t, f32x16 &s_cur, f32x16 &s_next) {
        constexpr int cur = decltype(parity)::value, nxt = cur ^ 1;
        const int k0 = k_begin + t * BN;
        if constexpr (PL) {
            // V of tile t + 1 over tile t - 1's (read by the last step's P.V), K of tile t + 2
            // over tile t's (read by the last step's scores)
            if (t + 1 < n_tiles) copy_tile(vimg, k0 + BN, Vh[nxt], Vl[nxt]);
            if (t + 2 < n_tiles) copy_tile(kimg, k0 + 2 * BN, Kh[cur], Kl[cur]);
        } else {
            if (t + 2 < n_tiles) load_k(k0 + 2 * BN);
            if (t + 1 < n_tiles) load_v(k0 + BN);
        }
        const bool need_cur = wave_needs(k0);
        const bool need_next = t + 1 < n_tiles && wave_needs(k0 + BN);
        if (need_cur) mask_and_max(s_cur, k0);
        if (need_cur && need_next) {
            s_next = qk_exp(nxt, s_cur);
        } else if (need_cur) {
            exp_sum(s_cur);
        } else if (need_next) {
            s_next = qk(nxt);
        }
        if (need_cur) pv(s_cur, cur);
        if constexpr (PL) {
            // tile t + 1's K (copied a step ago) and V in LDS; tile t + 2's K may still be on its way
            if (t + 2 < n_tiles) __builtin_amdgcn_s_waitcnt(vmcnt_only(IMG_LOADS));
            else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        } else {
            if (t + 2 < n_tiles) store_k(cur);
            if (t + 1 < n_tiles) store_v(nxt);
        }
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

hipError_t launch_flash_x3(const AttnArgs &a, int d, hipStream_t stream, int *grid_blocks) {
    if (a.k_img) { // tile images: row-major, d 64 or 128
        const int n_qblocks = (a.n_q + kFlashBM - 1) / kFlashBM;
        const int64_t blocks =
            a.heavy_first == 2 ? a.live_blocks : (int64_t)a.max_chunks * n_qblocks * a.n_batch * a.n_head;
        if (blocks > 0x7fffffffll || a.kt_stride || !a.v_img) return hipErrorInvalidValue;
        if (grid_blocks) *grid_blocks = (int)blocks;
        if (d == 64) flash_x3_kernel<64, false, true><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(a);
        else if (d == 128) flash_x3_kernel<128, false, true><<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(a);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    const int n_qblocks = (a.n_q + kFlashBM - 1) / kFlashBM;
    const int64_t blocks = a.heavy_first == 2 ? a.live_blocks : (int64_t)a.max_chunks * n_qblocks * a.n_batch * a.n_head;
    if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
    dim3 grid((unsigned)blocks);
    dim3 block(256);
    if (grid_blocks) *grid_blocks = (int)grid.x;
    const bool kt = a.kt_stride != 0;
#define ZWG_FLASH_X3(DD)                                                                                         \
    if (d == DD) {                                                                                               \
        if (kt) flash_x3_kernel<DD, true><<<grid, block, 0, stream>>>(a);                                        \
        else flash_x3_kernel<DD, false><<<grid, block, 0, stream>>>(a);                                          \
        return hipGetLastError();                                                                                \
    }
    ZWG_FLASH_X3(32)
    ZWG_FLASH_X3(64)
    ZWG_FLASH_X3(128)
#undef ZWG_FLASH_X3
    return hipErrorInvalidValue;
}

} // namespace zwg
