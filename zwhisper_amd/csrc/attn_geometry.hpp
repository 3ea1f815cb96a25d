// Kernel geometry and the key split, shared by the kernels, the merge pass and the host planner.
// Plain C++ (no HIP headers): the planner is also built on its own for the sanitizer tests.
#pragma once

namespace zwg {

// Flash (dense, MFMA) kernel geometry.
constexpr int kFlashWaves = 4;
constexpr int kFlashRowsPerWave = 32;
constexpr int kFlashBM = kFlashWaves * kFlashRowsPerWave; // query rows per workgroup
constexpr int kFlashBN = 32;                              // keys per MFMA tile

// Decode (split-K streaming) kernel geometry.
#ifndef ZWG_DECODE_TILE
#define ZWG_DECODE_TILE 256
#endif
constexpr int kDecodeThreads = 256;
constexpr int kDecodeTile = ZWG_DECODE_TILE; // keys per inner tile
#ifndef ZWG_DECODE_SHORT_TILE
#define ZWG_DECODE_SHORT_TILE 64
#endif
constexpr int kDecodeShortTile = ZWG_DECODE_SHORT_TILE; // row-major K: tile of short caches
constexpr int kDecodeMaxRows = 8; // heads-per-KV-group x queries a block can carry

// Key split of one work unit whose rows see keys [0, kv_hi): its W = ceil(kv_hi / tile) tiles are
// dealt into chunks of equal length (the last may be shorter), about tau = chunk_len / tile
// tiles each, at most max_chunks.  Returns the number of chunks (>= 1) and sets *chunk_keys to
// the chunk length in keys.  The kernels, the merge pass and the planner all split this way
// (constexpr, so the same function serves host and device code).
constexpr int unit_split(int kv_hi, int tile, int chunk_len, int max_chunks, int *chunk_keys) {
    const int w = (kv_hi + tile - 1) / tile;
    if (w <= 0) {
        *chunk_keys = tile;
        return 1;
    }
    const int tau = chunk_len / tile > 1 ? chunk_len / tile : 1;
    int nc = (w + tau / 2) / tau; // round(w / tau)
    nc = nc < 1 ? 1 : nc > max_chunks ? max_chunks : nc;
    const int lt = (w + nc - 1) / nc;
    *chunk_keys = lt * tile;
    return (w + lt - 1) / lt;
}

} // namespace zwg
