// C++ mirror of zwhisper's attention interface (src/ops.zig:464-605) over the gfx950 library.
//
// Same names, argument meaning and error behaviour as the Zig functions:
//   ops.q_block, ops.AttnShape, ops.attentionScratch / attentionScratchEx / attentionScratchKT,
//   ops.attentionEx, ops.attention.
// The reference asserts its preconditions (src/ops.zig:564, :568) and panics in safe builds;
// here a violated precondition or a device failure prints a message and aborts the same way.
// The pool and scratch arguments are accepted and not used: the work runs on the GPU, whose
// per-thread context (opened on first use) owns its own device memory.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>

namespace zw::ops {

// The reference's vector width on AVX-512 hosts (src/gemm.zig:15-24); it only sizes scratch.
constexpr std::size_t V = 16;
// Query rows per task (src/ops.zig:473).
constexpr std::size_t q_block = 64;

// Stand-in for ops.Pool (src/ops.zig:31): callers keep passing theirs; the GPU path ignores it.
struct Pool;

// ops.AttnShape (src/ops.zig:477-492).
struct AttnShape {
    std::size_t n_q;
    std::size_t n_kv;
    std::size_t n_head;
    std::size_t n_head_kv;
    std::size_t d;
    std::size_t q_stride;
    std::size_t kv_stride;
    std::size_t out_stride;
    bool causal;
    std::optional<std::size_t> kt_stride = std::nullopt;
};

// A Zig slice: pointer and length.
template <class T> struct Slice {
    T *ptr;
    std::size_t len;
};

std::size_t attentionScratchEx(std::size_t n_q, std::size_t n_kv, std::size_t n_head, std::size_t n_head_kv,
                               std::size_t d);
std::size_t attentionScratchKT(std::size_t n_q, std::size_t kt_stride, std::size_t n_head);
std::size_t attentionScratch(std::size_t n_q, std::size_t n_kv, std::size_t n_head, std::size_t n_state);

void attentionEx(Pool *pool, Slice<const float> q, Slice<const float> k, Slice<const float> v, AttnShape sh,
                 Slice<float> scratch, Slice<float> out);

void attention(Pool *pool, Slice<const float> q, Slice<const float> k, Slice<const float> v, std::size_t n_q,
               std::size_t n_kv, std::size_t n_state, std::size_t n_head, bool causal, Slice<float> scratch,
               Slice<float> out);

} // namespace zw::ops
