// Host planner of the attention calls: shape rules, work units, key splits and the workspace
// layout of the split partials.  Plain C++ (no HIP headers), so the planner is also built on its
// own, under the address / undefined-behaviour sanitizers (tests/cpp/test_plan_sanitize.cpp).
#pragma once

#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <string>

#include "attn_geometry.hpp"
#include "zw_gpu.h"

namespace zwg_planner {

constexpr uint64_t kDefaultWorkspace = 256ull << 20;
constexpr int kNumCUs = 256;
// Largest key split count: keeps chunk indices and partial-slot offsets small.
constexpr uint64_t kMaxChunks = 4096;
// Calls with more work units than this fill the machine without splitting keys.
constexpr uint64_t kMaxSplitUnitsHint = 1ull << 22;

// Planner tunables (compile-time).
#ifndef ZWG_DECODE_BLOCKS_PER_CU
#define ZWG_DECODE_BLOCKS_PER_CU 8 // decode grid size aimed at, per CU
#endif
#ifndef ZWG_DECODE_NOSPLIT_UNITS_PER_CU
#define ZWG_DECODE_NOSPLIT_UNITS_PER_CU 64 // no key split once units alone reach this many per CU
#endif
#ifndef ZWG_DECODE_NOSPLIT_TILES
#define ZWG_DECODE_NOSPLIT_TILES 0 // ... or when a unit has at most this many 256-key tiles
#endif
#ifndef ZWG_DECODE_SHORT_KV
#define ZWG_DECODE_SHORT_KV 512 // row-major decode calls up to this many keys use the short key tile
#endif
#ifndef ZWG_FLASH_BLOCKS_PER_CU
#define ZWG_FLASH_BLOCKS_PER_CU 2 // dense grid aimed at when keys are split, per CU
#endif
#ifndef ZWG_FLASH_CAUSAL_BLOCKS_PER_CU
#define ZWG_FLASH_CAUSAL_BLOCKS_PER_CU 2 // ... for causal calls, dispatched longest-first
#endif
// Key tiles an x3 dense split chunk is given at least: a small causal call (the 256-row prompt
// batches of a Qwen2.5-0.5B prefill) would otherwise be cut into chunks of 4 tiles whose fixed
// costs and merge outweigh the parallelism (8 calls of 256 rows: 156 us at 1, 149 at 6, 150 at 8,
// 179 at 12; the 2048-row call and tiny.en unchanged at 6).  The fp32 kernel keeps its finer
// split (its 2048-row prefill: 101 us at 5 tiles a chunk, 109 us held to 6).
#ifndef ZWG_FLASH_MIN_CHUNK_TILES
#define ZWG_FLASH_MIN_CHUNK_TILES 6
#endif
#ifndef ZWG_FLASH32_CAUSAL_BLOCKS_PER_CU
#define ZWG_FLASH32_CAUSAL_BLOCKS_PER_CU 6 // ... the same for the fp32 dense kernel (ZWG_DENSE_FP32)
#endif

// Largest head dim: the built kernels take 32, 64 and 128 (other dims up to 128 on zero-padded
// copies); above 128 a plain f32 kernel (attn_generic.hip) takes any multiple of 4 up to this.
constexpr int kMaxHeadDim = 1024;

// Shape rules: the reference's asserts (src/ops.zig:564, :568; causal needs n_kv >= n_q,
// src/ops.zig:534) plus this build's limits.
inline std::string check_shape(const zwg_attn_shape &s) {
    const uint64_t lim = 1ull << 30; // keeps every key and row index, plus a tile, within int32
    char buf[256];
    if (s.reserved != 0) return "shape.reserved must be 0";
    if (s.d == 0 || s.d % 4 != 0 || s.d > (uint64_t)kMaxHeadDim) {
        snprintf(buf, sizeof buf, "head dim d=%llu unsupported (this build: multiples of 4 up to %d)",
                 (unsigned long long)s.d, kMaxHeadDim);
        return buf;
    }
    if (s.n_head == 0 || s.n_head_kv == 0 || s.n_head % s.n_head_kv != 0) {
        snprintf(buf, sizeof buf, "n_head=%llu must be a positive multiple of n_head_kv=%llu",
                 (unsigned long long)s.n_head, (unsigned long long)s.n_head_kv);
        return buf;
    }
    if (s.n_q >= lim || s.n_kv >= lim || s.n_head >= lim) return "n_q, n_kv and n_head must be below 2^30";
    if (s.causal && s.n_kv < s.n_q) {
        snprintf(buf, sizeof buf, "causal attention needs n_kv >= n_q (n_kv=%llu, n_q=%llu)",
                 (unsigned long long)s.n_kv, (unsigned long long)s.n_q);
        return buf;
    }
    if (s.q_stride % 4 || s.kv_stride % 4 || s.out_stride % 4 || s.kt_stride % 4)
        return "q_stride, kv_stride, out_stride and kt_stride must be multiples of 4 floats";
    if (s.n_q > 1 && s.q_stride < s.n_head * s.d) return "q_stride is smaller than n_head * d";
    if (s.n_q > 1 && s.out_stride < s.n_head * s.d) return "out_stride is smaller than n_head * d";
    if (s.n_kv > 1 && s.kv_stride < s.n_head_kv * s.d) return "kv_stride is smaller than n_head_kv * d";
    if (s.kt_stride && s.kt_stride < s.n_kv) return "kt_stride is smaller than n_kv";
    return "";
}

inline std::string check_batch(const zwg_attn_shape &s, const zwg_batch &b) {
    if (b.n_batch == 0 || b.n_batch > 65535) return "n_batch must be in 1..65535";
    if (b.q_bstride % 4 || b.k_bstride % 4 || b.v_bstride % 4 || b.out_bstride % 4)
        return "batch strides must be multiples of 4 floats";
    if (s.n_head * b.n_batch > 0x7fffffffull) return "n_head * n_batch must be below 2^31";
    return "";
}

// The head dim the kernels run at: d itself for the built dims 32, 64 and 128, else the next
// of them, over zero-padded copies of the tensors (attn_pad.hip).
inline uint64_t kernel_d(uint64_t d) { return d <= 32 ? 32 : d <= 64 ? 64 : d <= 128 ? 128 : d; }

struct Plan {
    int kernel = 0; // 1 flash, 2 decode, 3 generic (head dims above 128)
    int rows_per_unit = 0;
    int split_tile = 0;
    int chunk_len = 0;
    int max_chunks = 1;
    int heavy_first = 0;
    int xcd_group = 0;
    uint64_t grid_blocks = 0;
    uint64_t ws_bytes = 0;
};

inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Split partials in the workspace: (max, sum) pairs [row][chunk][2], then, from the next 256-byte
// boundary (so the kernels' 16-byte partial stores and the merge's loads stay aligned), the sums
// [row][chunk][d].  Floats before part_o, and bytes of the whole layout:
inline uint64_t part_o_offset(uint64_t n_rows, uint64_t chunks) { return (2 * n_rows * chunks + 63) / 64 * 64; }
inline uint64_t split_ws_bytes(uint64_t n_rows, uint64_t chunks, uint64_t d) {
    return chunks > 1 ? (part_o_offset(n_rows, chunks) + n_rows * chunks * d) * sizeof(float) : 0;
}

// Chunks of about tau tiles that a unit of w tiles is split into (unit_split's count before
// the last chunk is trimmed): an upper bound on the chunks of any unit of at most w tiles.
inline uint64_t split_bound(uint64_t w, uint64_t tau) { return std::max<uint64_t>(1, (w + tau / 2) / tau); }

// Work units and key splits (unit_split deals a unit's key tiles into equal chunks of about
// tau tiles).  Decode: one unit per (item, KV head); keys split so the grid has ~8 workgroups
// per CU.  Dense: one unit per (item, head, 128-row q-block); when the units alone cannot fill
// the machine, keys are split so the workgroups are about equal in work, two per CU.  Causal
// calls (q-blocks of very unequal length) are always split, into about six workgroups per CU
// dispatched longest q-block first, so slots freed by short work keep the machine busy.
inline Plan make_plan(const zwg_attn_shape &s, const zwg_batch &b, uint64_t ws_cap, uint32_t dense_math) {
    Plan p;
    const uint64_t group = s.n_head / s.n_head_kv;
    const uint64_t n_rows_total = b.n_batch * s.n_head * s.n_q;
    uint64_t tile = 0, tau = 1, w_max = 1, units = 0;
    if (s.d > 128) {
        // one wavefront per query row, no key split (attn_generic.hip)
        p.kernel = 3;
        p.rows_per_unit = 1;
        p.split_tile = 64;
        p.chunk_len = 64;
        p.max_chunks = 1;
        p.grid_blocks = ceil_div(n_rows_total, 4);
        return p;
    }
    if (s.n_q * group <= (uint64_t)zwg::kDecodeMaxRows) {
        p.kernel = 2;
        p.rows_per_unit = (int)s.n_q;
        // row-major caches of at most ZWG_DECODE_SHORT_KV keys go in short tiles
        tile = !s.kt_stride && s.n_kv <= (uint64_t)ZWG_DECODE_SHORT_KV ? zwg::kDecodeShortTile : zwg::kDecodeTile;
        units = b.n_batch * s.n_head_kv;
        w_max = std::max<uint64_t>(1, ceil_div(s.n_kv, tile));
        uint64_t want_chunks =
            std::min<uint64_t>(w_max, std::max<uint64_t>(1, ceil_div(ZWG_DECODE_BLOCKS_PER_CU * kNumCUs, units)));
        // no split when the units already fill the machine, or are short enough that a merge
        // pass would cost more than the extra parallelism gains
        if (units >= (uint64_t)ZWG_DECODE_NOSPLIT_UNITS_PER_CU * kNumCUs || w_max <= ZWG_DECODE_NOSPLIT_TILES)
            want_chunks = 1;
        tau = ceil_div(w_max, want_chunks);
    } else {
        p.kernel = 1;
        const uint64_t BM = zwg::kFlashBM;
        tile = zwg::kFlashBN;
        p.rows_per_unit = (int)BM;
        const uint64_t n_qb = ceil_div(s.n_q, BM);
        units = n_qb * s.n_head * b.n_batch;
        // key tiles of every q-block (causal blocks stop at their diagonal)
        uint64_t tiles = 0;
        for (uint64_t qb = 0; qb < n_qb; ++qb) {
            const uint64_t q_end = std::min(s.n_q, (qb + 1) * BM);
            const uint64_t hi = s.causal ? s.n_kv - s.n_q + q_end : s.n_kv;
            tiles += ceil_div(hi, tile);
        }
        tiles *= s.n_head * b.n_batch;
        w_max = std::max<uint64_t>(1, ceil_div(s.n_kv, tile));
        const uint64_t causal_target =
            dense_math == ZWG_DENSE_FP32 ? ZWG_FLASH32_CAUSAL_BLOCKS_PER_CU : ZWG_FLASH_CAUSAL_BLOCKS_PER_CU;
        const uint64_t target = (uint64_t)(s.causal ? causal_target : ZWG_FLASH_BLOCKS_PER_CU) * kNumCUs;
        tau = w_max;
        if (s.causal || units < target)
            tau = std::min(w_max, std::max<uint64_t>(dense_math == ZWG_DENSE_FP32 ? 1 : ZWG_FLASH_MIN_CHUNK_TILES,
                                                     ceil_div(tiles, target)));
    }
    if (units > kMaxSplitUnitsHint) tau = w_max;
    uint64_t chunks = split_bound(w_max, tau);
    while (chunks > 1 && (split_ws_bytes(n_rows_total, chunks, kernel_d(s.d)) > ws_cap || chunks > kMaxChunks)) {
        ++tau;
        chunks = split_bound(w_max, tau);
    }
    p.chunk_len = (int)(tau * tile);
    p.max_chunks = (int)chunks;
    p.split_tile = (int)tile;
    p.grid_blocks = p.kernel == 2 ? chunks * s.n_head_kv * b.n_batch : chunks * units;
    p.ws_bytes = split_ws_bytes(n_rows_total, (uint64_t)p.max_chunks, kernel_d(s.d));
    p.heavy_first = p.kernel == 1 && s.causal;
    if (p.heavy_first && !b.n_kv_dev) {
        // one key count for every item: the grid holds only the (q-block, chunk, item*head)
        // triples with keys (dense_live_unit)
        const uint64_t BM = zwg::kFlashBM, n_qb = ceil_div(s.n_q, BM);
        uint64_t live = 0;
        for (uint64_t qb = 0; qb < n_qb; ++qb) {
            const uint64_t q_end = std::min(s.n_q, (qb + 1) * BM);
            int ck = 0;
            live += (uint64_t)zwg::unit_split((int)(s.n_kv - s.n_q + q_end), (int)tile, p.chunk_len, p.max_chunks, &ck);
        }
        p.grid_blocks = live * s.n_head * b.n_batch;
        p.heavy_first = 2;
    }
    // unsplit non-causal calls: each head's q-blocks on one XCD (measured: same time, 5x fewer
    // L2 misses on the base.en encoder); split ones keep the hardware order (measured faster)
    p.xcd_group = p.kernel == 1 && !s.causal && p.max_chunks == 1;
    return p;
}

} // namespace zwg_planner
