/*
 * oracle/attn_oracle.c — CPU oracle for zwhisper's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it.  The product
 * path (zwhisper_amd/, the HIP library) never links, imports or calls it.
 *
 * It is a plain-C restatement of the reference's f32 CPU attention, step for step:
 *
 *   ops.attentionEx ........ src/ops.zig:562-590   (ora_attention_ex)
 *   ops.attention .......... src/ops.zig:593-605   (ora_attention)
 *   AttnJob.transpose ...... src/ops.zig:505-515   (job_transpose)
 *   AttnJob.run ............ src/ops.zig:517-541   (job_run)
 *   attentionScratch* ...... src/ops.zig:545-560   (ora_attention_scratch*)
 *   gemm.pvBlock ........... src/gemm.zig:140-186  (pv_block)
 *   expVec ................. src/ops.zig:177-209   (exp_vec)
 *   scale .................. src/ops.zig:223-231   (scale_row)
 *   softmaxRow ............. src/ops.zig:442-462   (softmax_row)
 *   Pool ................... src/ops.zig:31-146    (ora_pool_*)
 *   small_op_macs .......... src/ops.zig:280
 *   q_block = 64 ........... src/ops.zig:473
 *   ops.linear (f16 w) ..... src/ops.zig:283-306, LinearJob :247-275  (ora_linear_f16)
 *   gemm.ntBlock ........... src/gemm.zig:117-137  (nt_block_f16)
 *   gemm.micro4x4/1x4/dot1.. src/gemm.zig:40-115   (micro4x4_f16, micro1x4_f16, dot1_f16)
 *   ops.linear (Q8 w) ...... src/ops.zig:283-306, gemm.ntBlockQ :336-351 (ora_linear_q8)
 *   gemm.Q8.quantize ....... src/gemm.zig:209-230  (ora_q8_quantize)
 *   gemm.dotQ / micro4x4Q .. src/gemm.zig:274-333  (dot_q8, micro4x4_q8)
 *   gemm.mc, nc ............ src/gemm.zig:27-28
 *   ops.layerNormEps ....... src/ops.zig:342-395, normRow :355-381 (ora_layer_norm)
 *   ops.gelu ............... src/ops.zig:310-340, geluScalar/geluVec :312-327 (ora_gelu)
 *   ops.rmsNorm ............ src/ops.zig:409-427 (ora_rms_norm)
 *   ops.siluMul ............ src/ops.zig:429-439, siluVec :429-432 (ora_silu_mul)
 *
 * V, the vector width, is 16 (the reference's value on AVX-512 hosts, src/gemm.zig:15-24):
 * it fixes the K padding (n_kv_pad), the column count of S and the split between
 * vectorised exp and the scalar tail in softmaxRow.  Zig's @mulAdd is a fused multiply-add;
 * here the same expressions are written as a*b+c and built with -ffp-contract=fast so the
 * compiler fuses them.  The arithmetic matches the reference to within FMA contraction
 * choices, which is far inside the parity tolerance (2e-4 abs).
 *
 * Parity pinning: every exported function is checked in tests/test_oracle.py against the
 * f64 closed form (oracle/naive.py), the reference's own test shapes (src/ops.zig:655-704,
 * src/gemm.zig:431-448, src/ops.zig:706-716), closed-form special cases and invariants, and
 * the committed golden fixtures under tests/golden/.
 */
#define _GNU_SOURCE
#include <linux/futex.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <sys/syscall.h>
#include <unistd.h>

#define V 16
#define Q_BLOCK 64
#define SMALL_OP_MACS ((size_t)1 << 16)

typedef float vf __attribute__((vector_size(V * sizeof(float))));

static inline vf vload(const float *p) {
    vf r;
    memcpy(&r, p, sizeof r);
    return r;
}
static inline void vstore(float *p, vf x) { memcpy(p, &x, sizeof x); }
static inline vf vsplat(float s) { return (vf){0} + s; }
static inline vf vmax(vf a, vf b) {
    vf r;
    for (int i = 0; i < V; ++i) r[i] = a[i] > b[i] ? a[i] : b[i];
    return r;
}
static inline vf vmin(vf a, vf b) {
    vf r;
    for (int i = 0; i < V; ++i) r[i] = a[i] < b[i] ? a[i] : b[i];
    return r;
}
static inline float hsum(vf x) {
    float s = 0;
    for (int i = 0; i < V; ++i) s += x[i];
    return s;
}
static inline float hmax(vf x) {
    float m = x[0];
    for (int i = 1; i < V; ++i) m = x[i] > m ? x[i] : m;
    return m;
}

/* ---------------------------------------------------------------------------------------
 * expVec (src/ops.zig:177-209): clamp to [-87.3, 88.3], fx = floor(x*log2e + 0.5),
 * r = x - fx*c1 - fx*c2 (two-constant ln2 split), degree-5 polynomial, y = y*r^2 + r + 1,
 * then scale by 2^fx built in the exponent bits.
 * ------------------------------------------------------------------------------------- */
static inline vf exp_vec(vf x_in) {
    const vf x = vmin(vmax(x_in, vsplat(-87.3f)), vsplat(88.3f));
    vf fx = x * vsplat(1.44269504088896341f) + vsplat(0.5f);
    for (int i = 0; i < V; ++i) fx[i] = floorf(fx[i]);
    vf r = x - fx * vsplat(0.693359375f);
    r = r - fx * vsplat(-2.12194440e-4f);
    vf y = vsplat(1.9875691500e-4f) * r + vsplat(1.3981999507e-3f);
    y = y * r + vsplat(8.3334519073e-3f);
    y = y * r + vsplat(4.1665795894e-2f);
    y = y * r + vsplat(1.6666665459e-1f);
    y = y * r + vsplat(5.0000001201e-1f);
    const vf r2 = r * r;
    y = y * r2 + r;
    y = y + vsplat(1.0f);
    vf scale_v;
    for (int i = 0; i < V; ++i) {
        const int32_t bits = ((int32_t)fx[i] + 127) << 23;
        memcpy(&scale_v[i], &bits, sizeof bits);
    }
    return y * scale_v;
}

/* scale (src/ops.zig:223-231) */
static inline void scale_row(float *x, size_t n, float a) {
    const vf av = vsplat(a);
    size_t i = 0;
    for (; i + V <= n; i += V) vstore(x + i, vload(x + i) * av);
    for (; i < n; ++i) x[i] *= a;
}

/* softmaxRow (src/ops.zig:442-462): vector max + scalar tail, vector exp + scalar @exp
 * tail, sum, multiply by 1/sum. */
static inline void softmax_row(float *x, size_t n) {
    vf mxv = vsplat(-INFINITY);
    size_t i = 0;
    for (; i + V <= n; i += V) mxv = vmax(mxv, vload(x + i));
    float mx = hmax(mxv);
    for (; i < n; ++i) mx = x[i] > mx ? x[i] : mx;
    const vf mv = vsplat(mx);
    vf sv = vsplat(0);
    i = 0;
    for (; i + V <= n; i += V) {
        const vf e = exp_vec(vload(x + i) - mv);
        vstore(x + i, e);
        sv += e;
    }
    float sum = hsum(sv);
    for (; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    scale_row(x, n, 1.0f / sum);
}

/* ---------------------------------------------------------------------------------------
 * gemm.pvBlock (src/gemm.zig:140-186): C[m][d] = P[m][t] . V[t][d], d a multiple of V.
 * Four P rows at a time against up to four V-vectors of the output row, FMA chain in t
 * order; a one-row tail path for m % 4 rows.
 * ------------------------------------------------------------------------------------- */
static inline void pv_block(const float *p, size_t ldp, const float *v, size_t ldv, float *c, size_t ldc,
                            size_t m, size_t t, size_t d) {
    const size_t nd = d / V;
    size_t i = 0;
    for (; i + 4 <= m; i += 4) {
        for (size_t dv = 0; dv < nd; dv += 4) {
            const size_t w = nd - dv < 4 ? nd - dv : 4;
            vf acc[4][4];
            for (int r = 0; r < 4; ++r)
                for (int q = 0; q < 4; ++q) acc[r][q] = vsplat(0);
            if (w == 4) {
                for (size_t tt = 0; tt < t; ++tt) {
                    const float *vrow = v + tt * ldv + dv * V;
                    const vf p0 = vsplat(p[(i + 0) * ldp + tt]);
                    const vf p1 = vsplat(p[(i + 1) * ldp + tt]);
                    const vf p2 = vsplat(p[(i + 2) * ldp + tt]);
                    const vf p3 = vsplat(p[(i + 3) * ldp + tt]);
                    for (int q = 0; q < 4; ++q) {
                        const vf vv = vload(vrow + q * V);
                        acc[0][q] = p0 * vv + acc[0][q];
                        acc[1][q] = p1 * vv + acc[1][q];
                        acc[2][q] = p2 * vv + acc[2][q];
                        acc[3][q] = p3 * vv + acc[3][q];
                    }
                }
            } else {
                for (size_t tt = 0; tt < t; ++tt) {
                    const float *vrow = v + tt * ldv + dv * V;
                    const vf p0 = vsplat(p[(i + 0) * ldp + tt]);
                    const vf p1 = vsplat(p[(i + 1) * ldp + tt]);
                    const vf p2 = vsplat(p[(i + 2) * ldp + tt]);
                    const vf p3 = vsplat(p[(i + 3) * ldp + tt]);
                    for (size_t q = 0; q < w; ++q) {
                        const vf vv = vload(vrow + q * V);
                        acc[0][q] = p0 * vv + acc[0][q];
                        acc[1][q] = p1 * vv + acc[1][q];
                        acc[2][q] = p2 * vv + acc[2][q];
                        acc[3][q] = p3 * vv + acc[3][q];
                    }
                }
            }
            for (int r = 0; r < 4; ++r)
                for (size_t q = 0; q < w; ++q) vstore(c + (i + r) * ldc + (dv + q) * V, acc[r][q]);
        }
    }
    for (; i < m; ++i) {
        float *out = c + i * ldc;
        memset(out, 0, d * sizeof(float));
        for (size_t tt = 0; tt < t; ++tt) {
            const vf s = vsplat(p[i * ldp + tt]);
            const float *vrow = v + tt * ldv;
            for (size_t q = 0; q < d; q += V) vstore(out + q, s * vload(vrow + q) + vload(out + q));
        }
    }
}

/* ---------------------------------------------------------------------------------------
 * Pool (src/ops.zig:31-146): one job at a time; workers spin 50k iterations on a
 * generation word, then futex-wait; tasks are claimed with an atomic fetch-add; the caller
 * joins in and waits for every worker's ack.
 * ------------------------------------------------------------------------------------- */
typedef struct ora_job {
    void *ctx;
    void (*run)(void *, size_t);
    size_t n;
    _Atomic size_t next;
} ora_job;

typedef struct ora_pool {
    pthread_t *threads;
    size_t n_workers;
    _Atomic uint32_t gen;
    _Atomic size_t acks;
    _Atomic(ora_job *) job;
    _Atomic int quit;
    _Atomic size_t sleepers;
} ora_pool;

static void futex_wait(_Atomic uint32_t *addr, uint32_t val) {
    syscall(SYS_futex, (uint32_t *)addr, FUTEX_WAIT_PRIVATE, val, NULL, NULL, 0);
}
static void futex_wake_all(_Atomic uint32_t *addr) {
    syscall(SYS_futex, (uint32_t *)addr, FUTEX_WAKE_PRIVATE, 0x7fffffff, NULL, NULL, 0);
}

static void pool_wait_for_gen(ora_pool *p, uint32_t seen) {
    uint32_t spins = 0;
    while (atomic_load_explicit(&p->gen, memory_order_acquire) == seen) {
        if (spins < 50000) {
            ++spins;
            __builtin_ia32_pause();
            continue;
        }
        atomic_fetch_add_explicit(&p->sleepers, 1, memory_order_acq_rel);
        if (atomic_load_explicit(&p->gen, memory_order_acquire) == seen) futex_wait(&p->gen, seen);
        atomic_fetch_sub_explicit(&p->sleepers, 1, memory_order_acq_rel);
    }
}

static void pool_bump_gen(ora_pool *p) {
    atomic_fetch_add_explicit(&p->gen, 1, memory_order_release);
    if (atomic_load_explicit(&p->sleepers, memory_order_acquire) > 0) futex_wake_all(&p->gen);
}

static void pool_drain(ora_job *job) {
    for (;;) {
        const size_t i = atomic_fetch_add_explicit(&job->next, 1, memory_order_acq_rel);
        if (i >= job->n) break;
        job->run(job->ctx, i);
    }
}

static void *pool_worker(void *arg) {
    ora_pool *p = arg;
    uint32_t seen = 0;
    for (;;) {
        pool_wait_for_gen(p, seen);
        seen = atomic_load_explicit(&p->gen, memory_order_acquire);
        if (atomic_load_explicit(&p->quit, memory_order_acquire)) return NULL;
        ora_job *job = atomic_load_explicit(&p->job, memory_order_acquire);
        if (job) pool_drain(job);
        atomic_fetch_add_explicit(&p->acks, 1, memory_order_acq_rel);
    }
}

/* n_threads includes the calling thread; 1 means no workers. */
ora_pool *ora_pool_new(size_t n_threads) {
    ora_pool *p = calloc(1, sizeof *p);
    if (!p) return NULL;
    p->n_workers = n_threads > 1 ? n_threads - 1 : 0;
    p->threads = calloc(p->n_workers ? p->n_workers : 1, sizeof(pthread_t));
    for (size_t i = 0; i < p->n_workers; ++i) pthread_create(&p->threads[i], NULL, pool_worker, p);
    return p;
}

void ora_pool_free(ora_pool *p) {
    if (!p) return;
    atomic_store_explicit(&p->quit, 1, memory_order_release);
    pool_bump_gen(p);
    for (size_t i = 0; i < p->n_workers; ++i) pthread_join(p->threads[i], NULL);
    free(p->threads);
    free(p);
}

size_t ora_pool_size(const ora_pool *p) { return p->n_workers + 1; }

static void pool_parallel_for(ora_pool *p, size_t n, void *ctx, void (*func)(void *, size_t)) {
    if (n == 0) return;
    if (p->n_workers == 0 || n == 1) {
        for (size_t i = 0; i < n; ++i) func(ctx, i);
        return;
    }
    ora_job job = {.ctx = ctx, .run = func, .n = n};
    atomic_init(&job.next, 0);
    atomic_store_explicit(&p->job, &job, memory_order_release);
    atomic_store_explicit(&p->acks, 0, memory_order_release);
    pool_bump_gen(p);
    pool_drain(&job);
    while (atomic_load_explicit(&p->acks, memory_order_acquire) < p->n_workers) __builtin_ia32_pause();
    atomic_store_explicit(&p->job, NULL, memory_order_release);
}

/* ---------------------------------------------------------------------------------------
 * Attention (src/ops.zig:464-605).
 * ------------------------------------------------------------------------------------- */

/* Mirrors AttnShape (src/ops.zig:477-492); kt_stride == 0 stands for Zig's null. */
typedef struct ora_shape {
    uint64_t n_q, n_kv, n_head, n_head_kv, d;
    uint64_t q_stride, kv_stride, out_stride;
    uint64_t kt_stride;
    uint32_t causal;
    uint32_t reserved;
} ora_shape;

typedef struct attn_job {
    const float *q, *k, *v;
    float *out;
    ora_shape sh;
    size_t n_kv_pad;
    float *kt;     /* [n_head_kv][d][n_kv_pad] */
    float *scores; /* per task: Q_BLOCK * n_kv_pad */
    size_t n_qblocks;
} attn_job;

/* AttnJob.transpose (src/ops.zig:505-515) */
static void job_transpose(void *raw, size_t h) {
    const attn_job *j = raw;
    const size_t d = j->sh.d;
    float *kt = j->kt + h * d * j->n_kv_pad;
    for (size_t t = 0; t < j->sh.n_kv; ++t) {
        const float *src = j->k + t * j->sh.kv_stride + h * d;
        for (size_t p = 0; p < d; ++p) kt[p * j->n_kv_pad + t] = src[p];
    }
    for (size_t p = 0; p < d; ++p)
        for (size_t t = j->sh.n_kv; t < j->n_kv_pad; ++t) kt[p * j->n_kv_pad + t] = 0;
}

/* AttnJob.run (src/ops.zig:517-541) */
static void job_run(void *raw, size_t task) {
    const attn_job *j = raw;
    const ora_shape sh = j->sh;
    const size_t d = sh.d;
    const size_t h = task / j->n_qblocks;
    const size_t hk = h / (sh.n_head / sh.n_head_kv);
    const size_t qb = task % j->n_qblocks;
    const size_t q0 = qb * Q_BLOCK;
    const size_t q1 = q0 + Q_BLOCK < sh.n_q ? q0 + Q_BLOCK : sh.n_q;
    const size_t m = q1 - q0;
    float *sc = j->scores + task * Q_BLOCK * j->n_kv_pad;
    const float *kt = j->kt + hk * d * j->n_kv_pad;
    const size_t cols = (sh.n_kv + V - 1) / V * V;
    pv_block(j->q + q0 * sh.q_stride + h * d, sh.q_stride, kt, j->n_kv_pad, sc, j->n_kv_pad, m, d, cols);
    const float scl = 1.0f / sqrtf((float)d);
    for (size_t i = 0; i < m; ++i) {
        float *row = sc + i * j->n_kv_pad;
        const size_t limit = sh.causal ? sh.n_kv - sh.n_q + q0 + i + 1 : sh.n_kv;
        scale_row(row, limit, scl);
        softmax_row(row, limit);
        memset(row + limit, 0, (cols - limit) * sizeof(float));
    }
    pv_block(sc, j->n_kv_pad, j->v + hk * d, sh.kv_stride, j->out + q0 * sh.out_stride + h * d, sh.out_stride, m,
             sh.n_kv, d);
}

/* attentionScratchEx (src/ops.zig:545-549) */
size_t ora_attention_scratch_ex(size_t n_q, size_t n_kv, size_t n_head, size_t n_head_kv, size_t d) {
    const size_t n_kv_pad = (n_kv + V - 1) / V * V;
    const size_t n_qblocks = (n_q + Q_BLOCK - 1) / Q_BLOCK;
    return n_head_kv * d * n_kv_pad + n_head * n_qblocks * Q_BLOCK * n_kv_pad;
}

/* attentionScratchKT (src/ops.zig:552-555) */
size_t ora_attention_scratch_kt(size_t n_q, size_t kt_stride, size_t n_head) {
    const size_t n_qblocks = (n_q + Q_BLOCK - 1) / Q_BLOCK;
    return n_head * n_qblocks * Q_BLOCK * kt_stride;
}

/* attentionScratch (src/ops.zig:558-560) */
size_t ora_attention_scratch(size_t n_q, size_t n_kv, size_t n_head, size_t n_state) {
    return ora_attention_scratch_ex(n_q, n_kv, n_head, n_head, n_state / n_head);
}

/* Checks the preconditions the reference asserts (src/ops.zig:564, :568) plus the ones its
 * usize arithmetic implies (causal needs n_kv >= n_q, src/ops.zig:534).  0 ok, 2 error. */
static int check_shape(const ora_shape *sh, size_t scratch_len) {
    if (sh->d == 0 || sh->d % V != 0) return 2;
    if (sh->n_head_kv == 0 || sh->n_head % sh->n_head_kv != 0) return 2;
    if (sh->causal && sh->n_kv < sh->n_q) return 2;
    if (sh->kt_stride && (sh->kt_stride < sh->n_kv || sh->kt_stride % V != 0)) return 2;
    const size_t n_kv_pad = sh->kt_stride ? sh->kt_stride : (sh->n_kv + V - 1) / V * V;
    const size_t n_qblocks = (sh->n_q + Q_BLOCK - 1) / Q_BLOCK;
    const size_t kt_len = sh->kt_stride ? 0 : sh->n_head_kv * sh->d * n_kv_pad;
    if (scratch_len < kt_len + sh->n_head * n_qblocks * Q_BLOCK * n_kv_pad) return 2;
    return 0;
}

/* attentionEx (src/ops.zig:562-590).  Returns 2 where the reference would trip an assert. */
int ora_attention_ex(ora_pool *pool, const float *q, const float *k, const float *v, const ora_shape *shp,
                     float *scratch, size_t scratch_len, float *out) {
    const ora_shape sh = *shp;
    if (check_shape(&sh, scratch_len)) return 2;
    const size_t n_kv_pad = sh.kt_stride ? sh.kt_stride : (sh.n_kv + V - 1) / V * V;
    const size_t n_qblocks = (sh.n_q + Q_BLOCK - 1) / Q_BLOCK;
    const size_t kt_len = sh.kt_stride ? 0 : sh.n_head_kv * sh.d * n_kv_pad;
    attn_job job = {
        .q = q,
        .k = k,
        .v = v,
        .out = out,
        .sh = sh,
        .n_kv_pad = n_kv_pad,
        .kt = sh.kt_stride ? (float *)k : scratch,
        .scores = scratch + kt_len,
        .n_qblocks = n_qblocks,
    };
    const int small = sh.n_q * sh.n_kv * sh.n_head * sh.d < SMALL_OP_MACS;
    if (!sh.kt_stride) {
        if (small || !pool) {
            for (size_t h = 0; h < sh.n_head_kv; ++h) job_transpose(&job, h);
        } else {
            pool_parallel_for(pool, sh.n_head_kv, &job, job_transpose);
        }
    }
    if (small || !pool) {
        for (size_t i = 0; i < sh.n_head * n_qblocks; ++i) job_run(&job, i);
    } else {
        pool_parallel_for(pool, sh.n_head * n_qblocks, &job, job_run);
    }
    return 0;
}

/* attention (src/ops.zig:593-605) */
int ora_attention(ora_pool *pool, const float *q, const float *k, const float *v, size_t n_q, size_t n_kv,
                  size_t n_state, size_t n_head, int causal, float *scratch, size_t scratch_len, float *out) {
    const ora_shape sh = {
        .n_q = n_q,
        .n_kv = n_kv,
        .n_head = n_head,
        .n_head_kv = n_head,
        .d = n_head ? n_state / n_head : 0,
        .q_stride = n_state,
        .kv_stride = n_state,
        .out_stride = n_state,
        .kt_stride = 0,
        .causal = causal ? 1u : 0u,
    };
    return ora_attention_ex(pool, q, k, v, &sh, scratch, scratch_len, out);
}

/* ---------------------------------------------------------------------------------------
 * Entry points for the oracle's own tests: the building blocks on their own.
 * ------------------------------------------------------------------------------------- */

/* expVec over n values (n a multiple of V). */
void ora_exp_vec(const float *x, float *y, size_t n) {
    for (size_t i = 0; i + V <= n; i += V) vstore(y + i, exp_vec(vload(x + i)));
}

void ora_softmax_row(float *x, size_t n) { softmax_row(x, n); }

void ora_pv_block(const float *p, size_t ldp, const float *v, size_t ldv, float *c, size_t ldc, size_t m, size_t t,
                  size_t d) {
    pv_block(p, ldp, v, ldv, c, ldc, m, t, d);
}

int ora_vector_width(void) { return V; }
int ora_q_block(void) { return Q_BLOCK; }

/* ---------------------------------------------------------------------------------------
 * ops.linear with f16 weights (src/ops.zig:283-306; src/gemm.zig:27-137).
 * out[i][o] = sum_p x[i][p] * w[o][p] (+ b[o]); w is IEEE binary16, widened per vector
 * (src/gemm.zig:34-38).
 * ------------------------------------------------------------------------------------- */

#define GEMM_MC 64  /* src/gemm.zig:27 */
#define GEMM_NC 128 /* src/gemm.zig:28 */

/* IEEE binary16 -> f32, exact (every f16 value is an f32 value). */
static inline float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (e == 0) { /* zero or subnormal: man * 2^-24 */
        const float f = (float)man * 0x1p-24f;
        return sign ? -f : f;
    }
    const uint32_t bits = e == 31 ? sign | 0x7f800000u | (man << 13) : sign | ((e + 112u) << 23) | (man << 13);
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static inline vf vload_h(const uint16_t *p) {
    float t[V];
    for (int i = 0; i < V; ++i) t[i] = h2f(p[i]);
    return vload(t);
}

/* 4x4 micro-kernel (src/gemm.zig:40-75): c[i][j] = dot(a_i, b_j) over k. */
static inline void micro4x4_f16(const float *a, size_t lda, const uint16_t *b, size_t ldb, size_t k, float *c,
                                size_t ldc) {
    vf acc[4][4];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) acc[i][j] = (vf){0};
    size_t p = 0;
    for (; p + V <= k; p += V) {
        vf va[4], vb[4];
        for (int i = 0; i < 4; ++i) va[i] = vload(a + i * lda + p);
        for (int j = 0; j < 4; ++j) vb[j] = vload_h(b + j * ldb + p);
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j) acc[i][j] = va[i] * vb[j] + acc[i][j];
    }
    float s[4][4];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) s[i][j] = hsum(acc[i][j]);
    for (; p < k; ++p)
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j) s[i][j] += a[i * lda + p] * h2f(b[j * ldb + p]);
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) c[i * ldc + j] = s[i][j];
}

/* 1x4 rows (src/gemm.zig:78-101). */
static inline void micro1x4_f16(const float *a, const uint16_t *b, size_t ldb, size_t k, float *c) {
    vf acc[4] = {{0}, {0}, {0}, {0}};
    size_t p = 0;
    for (; p + V <= k; p += V) {
        const vf va = vload(a + p);
        for (int j = 0; j < 4; ++j) acc[j] = va * vload_h(b + j * ldb + p) + acc[j];
    }
    float s[4];
    for (int j = 0; j < 4; ++j) s[j] = hsum(acc[j]);
    for (; p < k; ++p)
        for (int j = 0; j < 4; ++j) s[j] += a[p] * h2f(b[j * ldb + p]);
    for (int j = 0; j < 4; ++j) c[j] = s[j];
}

/* One row against one weight row (src/gemm.zig:106-113). */
static inline float dot1_f16(const float *a, const uint16_t *b, size_t k) {
    vf acc = (vf){0};
    size_t p = 0;
    for (; p + V <= k; p += V) acc = vload(a + p) * vload_h(b + p) + acc;
    float s = hsum(acc);
    for (; p < k; ++p) s += a[p] * h2f(b[p]);
    return s;
}

/* Rows [m0,m1) of a against weight rows [n0,n1) (src/gemm.zig:117-137). */
static void nt_block_f16(const float *a, size_t lda, const uint16_t *b, size_t ldb, float *c, size_t ldc, size_t m0,
                         size_t m1, size_t n0, size_t n1, size_t k) {
    size_t j = n0;
    for (; j + 4 <= n1; j += 4) {
        const uint16_t *bj = b + j * ldb;
        size_t i = m0;
        for (; i + 4 <= m1; i += 4) micro4x4_f16(a + i * lda, lda, bj, ldb, k, c + i * ldc + j, ldc);
        for (; i < m1; ++i) micro1x4_f16(a + i * lda, bj, ldb, k, c + i * ldc + j);
    }
    for (; j < n1; ++j)
        for (size_t i = m0; i < m1; ++i) c[i * ldc + j] = dot1_f16(a + i * lda, b + j * ldb, k);
}

typedef struct linear_job {
    const float *x;
    const uint16_t *w;   /* f16 weights, or NULL for int8 blocks */
    const int8_t *q;     /* int8 blocks [n][k] */
    const float *scales; /* [n][k / 32] */
    const float *b;
    float *out;
    size_t m, n, k, mb, nb, n_mblocks;
} linear_job;

static void nt_block_q8(const float *a, size_t lda, const int8_t *q, const float *scales, size_t k, float *c,
                        size_t ldc, size_t m0, size_t m1, size_t n0, size_t n1);

/* LinearJob.run (src/ops.zig:260-274): one (m-block, n-block) task, then its bias. */
static void linear_task(void *raw, size_t task) {
    const linear_job *j = raw;
    const size_t mi = task % j->n_mblocks, ni = task / j->n_mblocks;
    const size_t m0 = mi * j->mb, m1 = m0 + j->mb < j->m ? m0 + j->mb : j->m;
    const size_t n0 = ni * j->nb, n1 = n0 + j->nb < j->n ? n0 + j->nb : j->n;
    if (j->w)
        nt_block_f16(j->x, j->k, j->w, j->k, j->out, j->n, m0, m1, n0, n1, j->k);
    else
        nt_block_q8(j->x, j->k, j->q, j->scales, j->k, j->out, j->n, m0, m1, n0, n1);
    if (j->b)
        for (size_t i = m0; i < m1; ++i)
            for (size_t o = n0; o < n1; ++o) j->out[i * j->n + o] += j->b[o];
}

/* ops.linear (src/ops.zig:283-306): serial below small_op_macs, else m-blocks of mc rows and
 * n-blocks halved until there are at least 3 tasks per thread. */
static void linear_any(ora_pool *pool, const float *x, size_t m, size_t k, const uint16_t *w, const int8_t *q,
                       const float *scales, const float *b, size_t n, float *out) {
    linear_job job = {.x = x, .w = w, .q = q, .scales = scales, .b = b, .out = out, .m = m, .n = n, .k = k};
    if (m * n * k < SMALL_OP_MACS) {
        job.mb = m ? m : 1;
        job.nb = n;
        job.n_mblocks = 1;
        linear_task(&job, 0);
        return;
    }
    const size_t mb = m >= GEMM_MC ? GEMM_MC : m;
    size_t nb = GEMM_NC;
    const size_t n_mblocks = (m + mb - 1) / mb;
    const size_t want = ora_pool_size(pool) * 3;
    while (n_mblocks * ((n + nb - 1) / nb) < want && nb > 4) nb /= 2;
    job.mb = mb;
    job.nb = nb;
    job.n_mblocks = n_mblocks;
    pool_parallel_for(pool, n_mblocks * ((n + nb - 1) / nb), &job, linear_task);
}

void ora_linear_f16(ora_pool *pool, const float *x, size_t m, size_t k, const uint16_t *w, const float *b, size_t n,
                    float *out) {
    linear_any(pool, x, m, k, w, NULL, NULL, b, n, out);
}

/* ---------------------------------------------------------------------------------------
 * Int8 block weights (gemm.Q8, src/gemm.zig:188-351): q int8 [n][k], scales f32 [n][k / 32],
 * every block of 32 weights of a row scaled by one f32 (absmax / 127).
 * ------------------------------------------------------------------------------------- */

#define Q8_BLOCK 32 /* src/gemm.zig:194 */

/* Q8.quantize (src/gemm.zig:209-230) of an f32 [n][k] matrix (f16 weights widen exactly):
 * scale = amax / 127, q = clamp(round(v * (127 / amax)), -127, 127), rounding half away from
 * zero (Zig's @round). */
void ora_q8_quantize(const float *w, size_t n, size_t k, int8_t *q, float *scales) {
    const size_t nb = k / Q8_BLOCK;
    for (size_t i = 0; i < n; ++i)
        for (size_t b = 0; b < nb; ++b) {
            const float *src = w + i * k + b * Q8_BLOCK;
            float amax = 0;
            for (int t = 0; t < Q8_BLOCK; ++t) amax = fmaxf(amax, fabsf(src[t]));
            const float scale = amax / 127.0f;
            const float inv = amax > 0 ? 127.0f / amax : 0;
            scales[i * nb + b] = scale;
            for (int t = 0; t < Q8_BLOCK; ++t) {
                const float r = roundf(src[t] * inv);
                q[i * k + b * Q8_BLOCK + t] = (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
            }
        }
}

static inline vf vload_q(const int8_t *p) {
    float t[V];
    for (int i = 0; i < V; ++i) t[i] = (float)p[i];
    return vload(t);
}

/* dotQ (src/gemm.zig:280-293): per block t = sum of a*q over V-wide FMA chains, then
 * acc = t * scale + acc; one horizontal sum at the end. */
static inline float dot_q8(const float *a, const int8_t *q, const float *sc, size_t nb) {
    vf acc = (vf){0};
    for (size_t b = 0; b < nb; ++b) {
        vf t = (vf){0};
        for (size_t c = 0; c < Q8_BLOCK / V; ++c) {
            const size_t off = b * Q8_BLOCK + c * V;
            t = vload(a + off) * vload_q(q + off) + t;
        }
        acc = t * vsplat(sc[b]) + acc;
    }
    return hsum(acc);
}

/* micro4x4Q (src/gemm.zig:296-333): 4 rows of a against 4 int8 rows, blocks as dotQ. */
static inline void micro4x4_q8(const float *a, size_t lda, const int8_t *q, const float *scales, size_t k, size_t j,
                               float *c, size_t ldc) {
    const size_t nb = k / Q8_BLOCK;
    vf acc[4][4];
    for (int i = 0; i < 4; ++i)
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] = (vf){0};
    for (size_t b = 0; b < nb; ++b) {
        vf t[4][4];
        for (int i = 0; i < 4; ++i)
            for (int jj = 0; jj < 4; ++jj) t[i][jj] = (vf){0};
        for (size_t ch = 0; ch < Q8_BLOCK / V; ++ch) {
            const size_t off = b * Q8_BLOCK + ch * V;
            vf va[4], vq[4];
            for (int i = 0; i < 4; ++i) va[i] = vload(a + i * lda + off);
            for (int jj = 0; jj < 4; ++jj) vq[jj] = vload_q(q + (j + jj) * k + off);
            for (int i = 0; i < 4; ++i)
                for (int jj = 0; jj < 4; ++jj) t[i][jj] = va[i] * vq[jj] + t[i][jj];
        }
        for (int jj = 0; jj < 4; ++jj) {
            const vf sv = vsplat(scales[(j + jj) * nb + b]);
            for (int i = 0; i < 4; ++i) acc[i][jj] = t[i][jj] * sv + acc[i][jj];
        }
    }
    for (int i = 0; i < 4; ++i)
        for (int jj = 0; jj < 4; ++jj) c[i * ldc + jj] = hsum(acc[i][jj]);
}

/* ntBlockQ (src/gemm.zig:336-351): 4x4 tiles, then the row tail by dotQ per weight row, then the
 * column tail by dotQ. */
static void nt_block_q8(const float *a, size_t lda, const int8_t *q, const float *scales, size_t k, float *c,
                        size_t ldc, size_t m0, size_t m1, size_t n0, size_t n1) {
    const size_t nb = k / Q8_BLOCK;
    size_t j = n0;
    for (; j + 4 <= n1; j += 4) {
        size_t i = m0;
        for (; i + 4 <= m1; i += 4) micro4x4_q8(a + i * lda, lda, q, scales, k, j, c + i * ldc + j, ldc);
        for (; i < m1; ++i)
            for (size_t jj = 0; jj < 4; ++jj)
                c[i * ldc + j + jj] = dot_q8(a + i * lda, q + (j + jj) * k, scales + (j + jj) * nb, nb);
    }
    for (; j < n1; ++j)
        for (size_t i = m0; i < m1; ++i) c[i * ldc + j] = dot_q8(a + i * lda, q + j * k, scales + j * nb, nb);
}

/* ops.linear with Q8 weights; k must be a multiple of 32 (Q8.quantize's assertion). */
void ora_linear_q8(ora_pool *pool, const float *x, size_t m, size_t k, const int8_t *q, const float *scales,
                   const float *b, size_t n, float *out) {
    linear_any(pool, x, m, k, NULL, q, scales, b, n, out);
}

/* ---------------------------------------------------------------------------------------
 * Row-wise and elementwise ops of an encoder layer.  Zig's default float mode does not
 * contract a*b+c, so these functions are built with contraction off and use fmaf exactly where
 * the reference writes @mulAdd.
 * ------------------------------------------------------------------------------------- */

/* normRow (src/ops.zig:355-381) */
__attribute__((optimize("fp-contract=off"))) static void norm_row(const float *row, size_t n, const float *w,
                                                                   const float *b, float eps, float *o) {
    vf sv = vsplat(0);
    size_t i = 0;
    for (; i + V <= n; i += V) sv += vload(row + i);
    float sum = hsum(sv);
    for (; i < n; ++i) sum += row[i];
    const float mean = sum / (float)n;
    const vf mv = vsplat(mean);
    vf qv = vsplat(0);
    i = 0;
    for (; i + V <= n; i += V) {
        const vf d = vload(row + i) - mv;
        for (int e = 0; e < V; ++e) qv[e] = fmaf(d[e], d[e], qv[e]);
    }
    float sq = hsum(qv);
    for (; i < n; ++i) {
        const float d = row[i] - mean;
        sq += d * d;
    }
    const float inv = 1.0f / sqrtf(sq / (float)n + eps);
    const vf iv = vsplat(inv);
    i = 0;
    for (; i + V <= n; i += V) {
        const vf d = (vload(row + i) - mv) * iv;
        const vf wv = vload(w + i), bv = vload(b + i);
        vf r;
        for (int e = 0; e < V; ++e) r[e] = fmaf(d[e], wv[e], bv[e]);
        vstore(o + i, r);
    }
    for (; i < n; ++i) o[i] = (row[i] - mean) * inv * w[i] + b[i];
}

typedef struct {
    const float *x, *w, *b;
    float *out;
    size_t n, m, rows_per_task;
    float eps;
} norm_job;

static void norm_task(void *raw, size_t task) {
    const norm_job *j = raw;
    const size_t r0 = task * j->rows_per_task;
    const size_t r1 = r0 + j->rows_per_task < j->m ? r0 + j->rows_per_task : j->m;
    for (size_t i = r0; i < r1; ++i) norm_row(j->x + i * j->n, j->n, j->w, j->b, j->eps, j->out + i * j->n);
}

/* layerNormEps (src/ops.zig:388-395): 64 rows per task */
void ora_layer_norm(ora_pool *pool, const float *x, size_t m, size_t n, const float *w, const float *b, float eps,
                    float *out) {
    norm_job j = {x, w, b, out, n, m, 64, eps};
    pool_parallel_for(pool, (m + 63) / 64, &j, norm_task);
}

/* ops.rmsNorm (src/ops.zig:409-427), serial as the reference runs it: per row the sum of squares
 * in V lanes (fma), reduced, plus the scalar tail; inv = 1 / sqrt(ss / n + eps); out = row * inv
 * * w, multiplied left to right. */
void ora_rms_norm(const float *x, size_t m, size_t n, const float *w, float eps, float *out) {
    for (size_t i = 0; i < m; ++i) {
        const float *row = x + i * n;
        float *o = out + i * n;
        vf sv = (vf){0};
        size_t j = 0;
        for (; j + V <= n; j += V) {
            const vf v = vload(row + j);
            sv = v * v + sv;
        }
        float ss = hsum(sv);
        for (; j < n; ++j) ss += row[j] * row[j];
        const float inv = 1.0f / sqrtf(ss / (float)n + eps);
        j = 0;
        for (; j + V <= n; j += V) {
            const vf r = vload(row + j) * vsplat(inv);
            vstore(o + j, r * vload(w + j));
        }
        for (; j < n; ++j) {
            const float r = row[j] * inv;
            o[j] = r * w[j];
        }
    }
}

/* ops.siluMul (src/ops.zig:429-439): gate = gate / (1 + expVec(-gate)) * up over V-wide vectors,
 * the tail with exp; serial as the reference runs it. */
__attribute__((optimize("fp-contract=off"))) void ora_silu_mul(float *gate, const float *up, size_t len) {
    size_t i = 0;
    const vf one = vsplat(1.0f);
    for (; i + V <= len; i += V) {
        const vf g = vload(gate + i);
        const vf s = g / (one + exp_vec(-g));
        vstore(gate + i, s * vload(up + i));
    }
    for (; i < len; ++i) gate[i] = gate[i] / (1.0f + expf(-gate[i])) * up[i];
}

/* geluScalar (src/ops.zig:312-315): std.math.tanh */
__attribute__((optimize("fp-contract=off"))) static float gelu_scalar(float x) {
    const float c = 0.7978845608028654f;
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

/* geluVec (src/ops.zig:317-327): tanh(u) = 1 - 2 / (1 + expVec(2u)) */
__attribute__((optimize("fp-contract=off"))) static vf gelu_vec(vf x) {
    const vf c = vsplat(0.7978845608028654f), k = vsplat(0.044715f), one = vsplat(1.0f), two = vsplat(2.0f),
             half = vsplat(0.5f);
    const vf u = c * (x + k * x * x * x);
    const vf t = one - two / (one + exp_vec(two * u));
    return half * x * (one + t);
}

typedef struct {
    float *x;
    size_t len, chunk;
} gelu_job;

static void gelu_task(void *raw, size_t task) {
    const gelu_job *j = raw;
    const size_t a = task * j->chunk, e = a + j->chunk < j->len ? a + j->chunk : j->len;
    size_t i = a;
    for (; i + V <= e; i += V) vstore(j->x + i, gelu_vec(vload(j->x + i)));
    for (; i < e; ++i) j->x[i] = gelu_scalar(j->x[i]);
}

/* ops.gelu (src/ops.zig:335-340): in place, tasks of 32 Ki elements */
void ora_gelu(ora_pool *pool, float *x, size_t len) {
    gelu_job j = {x, len, 32 * 1024};
    pool_parallel_for(pool, (len + j.chunk - 1) / j.chunk, &j, gelu_task);
}
