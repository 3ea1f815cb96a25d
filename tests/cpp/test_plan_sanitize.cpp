// The host planner (zwhisper_amd/csrc/attn_plan.hpp) built on its own, with no GPU, under the
// address and undefined-behaviour sanitizers: random shapes and batches through the shape rules
// and make_plan, every accepted plan checked against the invariants the kernels and the merge
// pass rely on (chunk length a multiple of the tile, at most max_chunks non-empty chunks per unit
// covering its keys exactly, partials within the workspace, the grid size).  Built and run by
// tests/test_sanitizers.py.
#include <cstdio>
#include <cstdlib>
#include <random>

#include "attn_plan.hpp"

using namespace zwg_planner;

static int g_fail = 0;
#define CHECK(cond, ...)                                                                                           \
    do {                                                                                                           \
        if (!(cond)) {                                                                                             \
            std::fprintf(stderr, "FAIL %s:%d: %s | ", __FILE__, __LINE__, #cond);                                \
            std::fprintf(stderr, __VA_ARGS__);                                                                     \
            std::fprintf(stderr, "\n");                                                                            \
            if (++g_fail > 20) std::exit(1);                                                                       \
        }                                                                                                          \
    } while (0)

// Every key range [0, kv_hi) of a unit must split into 1..max_chunks chunks that cover it.
static void check_unit(const Plan &p, int kv_hi, const zwg_attn_shape &s) {
    int keys = 0;
    const int n = zwg::unit_split(kv_hi, p.split_tile, p.chunk_len, p.max_chunks, &keys);
    CHECK(n >= 1 && n <= p.max_chunks, "kv_hi %d chunks %d max %d (n_q %llu n_kv %llu)", kv_hi, n, p.max_chunks,
          (unsigned long long)s.n_q, (unsigned long long)s.n_kv);
    CHECK(keys % p.split_tile == 0 && keys > 0, "chunk keys %d tile %d", keys, p.split_tile);
    if (kv_hi > 0) CHECK((long long)(n - 1) * keys < kv_hi && kv_hi <= (long long)n * keys, "cover %d: %d x %d", kv_hi, n, keys);
}

int main() {
    std::mt19937_64 rng(20261202);
    auto pick = [&](std::initializer_list<uint64_t> v) { return *(v.begin() + rng() % v.size()); };
    long accepted = 0, rejected = 0;
    for (int it = 0; it < 40000; ++it) {
        zwg_attn_shape s{};
        const uint64_t big = rng() % 8 == 0;
        s.n_q = big ? rng() % (1ull << 31) : pick({0, 1, 2, 3, 7, 64, 127, 128, 129, 300, 1500, 2048, 4096});
        s.n_kv = big ? rng() % (1ull << 31) : pick({0, 1, 5, 17, 90, 255, 256, 257, 448, 1500, 2048, 4096, 32768});
        s.n_head_kv = pick({1, 2, 4, 8});
        s.n_head = s.n_head_kv * pick({1, 2, 6, 7});
        s.d = pick({0, 4, 16, 32, 48, 64, 100, 128, 132, 256, 1024, 1028});
        s.causal = rng() % 2;
        const uint64_t hd = s.n_head * s.d, kvd = s.n_head_kv * s.d;
        s.q_stride = hd + 4 * (rng() % 3);
        s.out_stride = hd + 4 * (rng() % 3);
        s.kv_stride = kvd + 4 * (rng() % 3);
        s.kt_stride = rng() % 2 ? (s.n_kv + 3) / 4 * 4 + 4 * (rng() % 3) : 0;
        zwg_batch b{};
        b.n_batch = pick({1, 2, 16, 32, 64, 300, 65535, 70000});
        const uint64_t cap = pick({0, 1, 4096, 1ull << 20, 64ull << 20, 256ull << 20});
        const uint32_t mode = rng() % 2 ? ZWG_DENSE_FP32 : ZWG_DENSE_X3;
        std::string msg = check_shape(s);
        if (msg.empty()) msg = check_batch(s, b);
        if (!msg.empty()) {
            ++rejected;
            continue;
        }
        ++accepted;
        const Plan p = make_plan(s, b, cap, mode);
        CHECK(p.kernel == 1 || p.kernel == 2 || p.kernel == 3, "kernel %d", p.kernel);
        if (p.kernel == 3) { // head dims above 128: one wavefront per row, unsplit
            CHECK(s.d > 128 && p.max_chunks == 1 && p.ws_bytes == 0, "f32 kernel plan");
            CHECK(p.grid_blocks == ceil_div(b.n_batch * s.n_head * s.n_q, 4), "f32 kernel grid");
            continue;
        }
        CHECK(s.d <= 128, "head dims above 128 take the f32 kernel");
        CHECK(p.split_tile > 0 && p.chunk_len > 0 && p.chunk_len % p.split_tile == 0, "chunk_len %d tile %d", p.chunk_len,
              p.split_tile);
        CHECK(p.max_chunks >= 1 && (uint64_t)p.max_chunks <= kMaxChunks, "max_chunks %d", p.max_chunks);
        const uint64_t rows = b.n_batch * s.n_head * s.n_q;
        CHECK(p.ws_bytes == split_ws_bytes(rows, (uint64_t)p.max_chunks, kernel_d(s.d)), "ws bytes");
        CHECK(kernel_d(s.d) >= s.d && (kernel_d(s.d) == 32 || kernel_d(s.d) == 64 || kernel_d(s.d) == 128), "kernel d");
        CHECK(p.max_chunks == 1 || p.ws_bytes <= cap, "partials %llu over the workspace %llu",
              (unsigned long long)p.ws_bytes, (unsigned long long)cap);
        if (p.max_chunks > 1) CHECK(part_o_offset(rows, (uint64_t)p.max_chunks) % 64 == 0, "part_o alignment");
        if (p.kernel == 2) {
            CHECK(s.n_q * (s.n_head / s.n_head_kv) <= (uint64_t)zwg::kDecodeMaxRows, "decode rows");
            CHECK(p.grid_blocks == (uint64_t)p.max_chunks * s.n_head_kv * b.n_batch, "decode grid");
            // per-item counts may be anything up to the capacity
            for (uint64_t kv : {uint64_t(0), uint64_t(1), s.n_kv / 3, s.n_kv / 2 + 1, s.n_kv})
                if (kv <= s.n_kv) check_unit(p, (int)kv, s);
        } else {
            const uint64_t n_qb = ceil_div(s.n_q, zwg::kFlashBM);
            if (p.heavy_first == 2) {
                uint64_t live = 0;
                for (uint64_t qb = 0; qb < n_qb; ++qb) {
                    int ck = 0;
                    live += (uint64_t)zwg::unit_split((int)(s.n_kv - s.n_q + std::min(s.n_q, (qb + 1) * zwg::kFlashBM)),
                                                      p.split_tile, p.chunk_len, p.max_chunks, &ck);
                }
                CHECK(p.grid_blocks == live * s.n_head * b.n_batch, "live dense grid");
            } else {
                CHECK(p.grid_blocks == (uint64_t)p.max_chunks * n_qb * s.n_head * b.n_batch, "dense grid");
            }
            for (uint64_t qb : {uint64_t(0), n_qb / 2, n_qb ? n_qb - 1 : 0}) {
                const uint64_t q_end = std::min(s.n_q, (qb + 1) * zwg::kFlashBM);
                const uint64_t hi = s.causal ? s.n_kv - s.n_q + q_end : s.n_kv;
                check_unit(p, (int)hi, s);
            }
        }
    }
    std::printf("planner: %ld plans checked, %ld shapes rejected, %d failures\n", accepted, rejected, g_fail);
    if (g_fail == 0) std::printf("ok\n");
    return g_fail ? 1 : 0;
}
