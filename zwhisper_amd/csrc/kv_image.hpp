// K and V "tile images": the layout in which the dense x3 attention kernel (attn_flash_x3.hip)
// holds a 32-key tile of one (batch item, KV head) in LDS -- f16 hi and lo planes of the f32
// values (hi = f16(x), lo = f16(x - hi)), 16-byte chunks XOR-swizzled by row -- laid out in HBM
// tile after tile.  The encoder layer's K and V projections write their outputs in this layout
// (the linear kernel's image epilogue), so its attention copies each tile into LDS as it is, with
// no f32 loads and no split: the same f16 terms the kernel would have formed from f32 K and V, so
// the results are the same bit for bit.
//
//   image of (item, head) = tiles blocks; block t = [hi plane: 32 x D][lo plane: 32 x D] halves
//   K plane:   row = key of the tile, D halves, chunk c (8 halves) of row r at c ^ ((r / (128 / D))
//              mod (D / 8))
//   V^T plane: row = dim, 32 halves (key positions), chunk c of row d at c ^ ((d / 4) mod 4); key j
//              sits at position j with bits 2 and 3 swapped (the P.V operand order)
// Keys past the item's last key in its last tile (padding) hold zeros.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zwg_img {

constexpr int kTileKeys = 32;

// K plane element (key, dim) of a D-dim tile
__host__ __device__ inline int k_at(int key, int dim, int D) {
    const int C = D / 8, R = 128 / D > 0 ? 128 / D : 1;
    return key * D + ((((dim >> 3) ^ ((key / R) & (C - 1))) << 3) | (dim & 7));
}
template <int D>
__host__ __device__ inline int k_at(int key, int dim) {
    constexpr int C = D / 8, R = 128 / D > 0 ? 128 / D : 1;
    return key * D + ((((dim >> 3) ^ ((key / R) & (C - 1))) << 3) | (dim & 7));
}
// V^T plane position of a key: bits 2 and 3 swapped (keys 4..7 <-> 8..11 of every 16)
__host__ __device__ inline int v_pos(int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); }
// V^T plane element (dim, pos)
__host__ __device__ inline int v_at(int dim, int pos) {
    return dim * kTileKeys + ((((pos >> 3) ^ ((dim >> 2) & 3)) << 3) | (pos & 7));
}
// halves of one tile block (both planes), and the block of tile t of image `ih` (item * heads + head)
__host__ __device__ inline int64_t block_halves(int D) { return 2ll * kTileKeys * D; }
__host__ __device__ inline int64_t block_offset(int64_t ih, int tiles, int t, int D) {
    return (ih * tiles + t) * block_halves(D);
}

typedef _Float16 img_half4 __attribute__((ext_vector_type(4)));
typedef float img_f32x4 __attribute__((ext_vector_type(4)));

// Store the values of keys key0 .. key0 + 3 (key0 % 4 == 0, one item) of column `dim` of head `h`
// from rows row0 .. row0 + 3 of a projection's output: rows are (item, key) with n_ctx keys per
// item (n_ctx % 4 == 0), columns (head, dim).  kind 1: K image, 2: V image.  The quad that ends an
// item also writes the zeros of its last tile's padding keys for these columns.  Kind 1 exchanges
// values within quads of lanes: the four lanes of a quad (lanes 4i .. 4i + 3) must hold dims
// 4c .. 4c + 3 of the same rows, in order, and call together.
__device__ inline void store_quad(_Float16 *img, int kind, int row0, int h, int dim, img_f32x4 v, int n_ctx, int D,
                                  int heads, int tiles) {
    const int item = row0 / n_ctx, key0 = row0 - item * n_ctx;
    const int t = key0 >> 5, kk = key0 & 31;
    _Float16 *hi = img + block_offset((int64_t)item * heads + h, tiles, t, D);
    _Float16 *lo = hi + kTileKeys * D;
    img_half4 vh, vl;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        vh[e] = (_Float16)v[e];
        vl[e] = (_Float16)(v[e] - (float)vh[e]);
    }
    const bool last = key0 + 4 == n_ctx && (n_ctx & 31) != 0;
    if (kind == 1) {
        // The quad of lanes holding dims 4c .. 4c + 3 (dim % 4 = the lane's place q in its quad)
        // transposes its 4 x 4 block with DPP quad permutes, so lane q then holds dims 4c .. 4c + 3 of
        // key key0 + q: 8-byte rows of the K plane.  Round r: each lane sends its key (q + r) % 4 and
        // receives the key q of the lane (q - r) % 4, i.e. dim 4c + (q - r) % 4 of its own key.
        const int q = dim & 3;
        // (bit casts of scalar copies: this compiler's __builtin_bit_cast of a vector element
        // expression reads element 0 whatever the index)
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const _Float16 eh = vh[e], el = vl[e];
            pk[e] = (uint32_t)__builtin_bit_cast(uint16_t, eh) | ((uint32_t)__builtin_bit_cast(uint16_t, el) << 16);
        }
        auto pick = [&](int i) { return i == 0 ? pk[0] : i == 1 ? pk[1] : i == 2 ? pk[2] : pk[3]; };
        uint32_t got[4];
        got[0] = pick(q);
        // quad_perm controls: lane q reads lane (q - r) % 4
        got[1] = (uint32_t)__builtin_amdgcn_mov_dpp((int)pick((q + 1) & 3), 0x93, 0xf, 0xf, true);
        got[2] = (uint32_t)__builtin_amdgcn_mov_dpp((int)pick((q + 2) & 3), 0x4e, 0xf, 0xf, true);
        got[3] = (uint32_t)__builtin_amdgcn_mov_dpp((int)pick((q + 3) & 3), 0x39, 0xf, 0xf, true);
        img_half4 th, tl; // dims 4c + e of key key0 + q: received in round (q - e) % 4
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = (q - e) & 3;
            const uint32_t u = r == 0 ? got[0] : r == 1 ? got[1] : r == 2 ? got[2] : got[3];
            th[e] = __builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
            tl[e] = __builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
        }
        const int at = k_at(kk + q, dim - q, D);
        *reinterpret_cast<img_half4 *>(hi + at) = th;
        *reinterpret_cast<img_half4 *>(lo + at) = tl;
        if (last)
            for (int kp = (n_ctx & 31) + q; kp < kTileKeys; kp += 4) {
                const int at0 = k_at(kp, dim - q, D);
                *reinterpret_cast<img_half4 *>(hi + at0) = (img_half4){0, 0, 0, 0};
                *reinterpret_cast<img_half4 *>(lo + at0) = (img_half4){0, 0, 0, 0};
            }
    } else {
        const int at = v_at(dim, v_pos(kk));
        *reinterpret_cast<img_half4 *>(hi + at) = vh;
        *reinterpret_cast<img_half4 *>(lo + at) = vl;
        if (last)
            for (int kp = n_ctx & 31; kp < kTileKeys; kp += 4) {
                const int at0 = v_at(dim, v_pos(kp));
                *reinterpret_cast<img_half4 *>(hi + at0) = (img_half4){0, 0, 0, 0};
                *reinterpret_cast<img_half4 *>(lo + at0) = (img_half4){0, 0, 0, 0};
            }
    }
}

} // namespace zwg_img
