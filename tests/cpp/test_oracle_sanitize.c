/* The CPU oracle (oracle/attn_oracle.c, test infrastructure) under the address / undefined-
 * behaviour sanitizers and, in a second build, the thread sanitizer: attention on the reference
 * test's shape and on GQA / transposed-key / decode shapes, against a double-precision triple
 * loop, and every result on a pool of 4 threads equal bit for bit to 1 thread (the futex Pool,
 * src/ops.zig:25-146); the f16 and int8 linear layers, layer norm and GELU through the pool too.
 * Built and run by tests/test_sanitizers.py. */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct ora_pool ora_pool;
typedef struct ora_shape {
    uint64_t n_q, n_kv, n_head, n_head_kv, d;
    uint64_t q_stride, kv_stride, out_stride;
    uint64_t kt_stride;
    uint32_t causal;
    uint32_t reserved;
} ora_shape;
ora_pool *ora_pool_new(size_t n_threads);
void ora_pool_free(ora_pool *p);
size_t ora_attention_scratch_ex(size_t n_q, size_t n_kv, size_t n_head, size_t n_head_kv, size_t d);
size_t ora_attention_scratch_kt(size_t n_q, size_t kt_stride, size_t n_head);
int ora_attention_ex(ora_pool *pool, const float *q, const float *k, const float *v, const ora_shape *sh, float *scratch,
                     size_t scratch_len, float *out);
void ora_linear_f16(ora_pool *pool, const float *x, size_t m, size_t k, const uint16_t *w, const float *b, size_t n,
                    float *out);
void ora_q8_quantize(const float *w, size_t n, size_t k, int8_t *q, float *scales);
void ora_linear_q8(ora_pool *pool, const float *x, size_t m, size_t k, const int8_t *q, const float *scales,
                   const float *b, size_t n, float *out);
void ora_layer_norm(ora_pool *pool, const float *x, size_t m, size_t n, const float *w, const float *b, float eps,
                    float *out);
void ora_gelu(ora_pool *pool, float *x, size_t len);

static int fails = 0;
static uint64_t rng_state = 0x5A57;
static float urand(void) {
    rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
    return (float)((rng_state >> 40) * (1.0 / 16777216.0)) - 0.5f;
}
static float *randv(size_t n) {
    float *p = malloc((n ? n : 1) * sizeof(float));
    for (size_t i = 0; i < n; ++i) p[i] = urand();
    return p;
}

/* out = softmax(scale q.k + mask) v per head, in double */
static void naive(const float *q, const float *k, const float *v, const ora_shape *s, double *out) {
    const double scale = (double)(1.0f / sqrtf((float)s->d));
    double *sc = malloc((s->n_kv ? s->n_kv : 1) * sizeof(double));
    for (size_t h = 0; h < s->n_head; ++h) {
        const size_t hk = h / (s->n_head / s->n_head_kv);
        for (size_t i = 0; i < s->n_q; ++i) {
            double mx = -INFINITY;
            const size_t lim = s->causal ? s->n_kv - s->n_q + i + 1 : s->n_kv;
            for (size_t j = 0; j < lim; ++j) {
                double acc = 0;
                for (size_t p = 0; p < s->d; ++p) {
                    const float kv = s->kt_stride ? k[(hk * s->d + p) * s->kt_stride + j] : k[j * s->kv_stride + hk * s->d + p];
                    acc += (double)q[i * s->q_stride + h * s->d + p] * kv;
                }
                sc[j] = acc * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            double sum = 0;
            for (size_t j = 0; j < lim; ++j) sum += (sc[j] = exp(sc[j] - mx));
            for (size_t p = 0; p < s->d; ++p) {
                double acc = 0;
                for (size_t j = 0; j < lim; ++j) acc += sc[j] * v[j * s->kv_stride + hk * s->d + p];
                out[i * s->out_stride + h * s->d + p] = lim ? acc / sum : 0.0;
            }
        }
    }
    free(sc);
}

static void attention_case(ora_pool *p1, ora_pool *p4, ora_shape s, const char *name) {
    const size_t kvd = s.n_head_kv * s.d;
    const size_t q_len = s.n_q * s.q_stride, v_len = s.n_kv * s.kv_stride;
    const size_t k_len = s.kt_stride ? kvd * s.kt_stride : v_len;
    const size_t o_len = s.n_q * s.out_stride;
    float *q = randv(q_len), *k = randv(k_len), *v = randv(v_len);
    const size_t scr = s.kt_stride ? ora_attention_scratch_kt(s.n_q, s.kt_stride, s.n_head)
                                   : ora_attention_scratch_ex(s.n_q, s.n_kv, s.n_head, s.n_head_kv, s.d);
    float *scratch = malloc((scr ? scr : 1) * sizeof(float));
    float *o1 = calloc(o_len, sizeof(float)), *o4 = calloc(o_len, sizeof(float));
    double *ref = calloc(o_len, sizeof(double));
    if (ora_attention_ex(p1, q, k, v, &s, scratch, scr, o1) || ora_attention_ex(p4, q, k, v, &s, scratch, scr, o4)) {
        printf("FAIL %s: rejected\n", name);
        ++fails;
    }
    naive(q, k, v, &s, ref);
    double err = 0;
    for (size_t i = 0; i < o_len; ++i) err = fmax(err, fabs(o1[i] - ref[i]));
    if (memcmp(o1, o4, o_len * sizeof(float)) || err > 1e-4) {
        printf("FAIL %s: max abs %.3e, 1 vs 4 threads %s\n", name, err, memcmp(o1, o4, o_len * sizeof(float)) ? "differ" : "equal");
        ++fails;
    }
    free(q), free(k), free(v), free(scratch), free(o1), free(o4), free(ref);
}

int main(void) {
    ora_pool *p1 = ora_pool_new(1), *p4 = ora_pool_new(4);
    /* the reference's own test shape (src/ops.zig:655-704), both mask modes */
    attention_case(p1, p4, (ora_shape){70, 90, 2, 2, 32, 64, 64, 64, 0, 0, 0}, "ref noncausal");
    attention_case(p1, p4, (ora_shape){70, 90, 2, 2, 32, 64, 64, 64, 0, 1, 0}, "ref causal");
    attention_case(p1, p4, (ora_shape){130, 140, 14, 2, 64, 896, 128, 896, 144, 1, 0}, "gqa transposed k");
    attention_case(p1, p4, (ora_shape){1, 300, 12, 2, 128, 1536, 256, 1536, 304, 1, 0}, "decode d128");
    attention_case(p1, p4, (ora_shape){33, 47, 2, 2, 32, 96, 80, 72, 0, 0, 0}, "strided rows");

    /* linear layers, layer norm, GELU through both pools */
    const size_t m = 37, kk = 96, n = 70;
    float *x = randv(m * kk), *wf = randv(n * kk), *bias = randv(n);
    uint16_t *w16 = malloc(n * kk * sizeof(uint16_t));
    for (size_t i = 0; i < n * kk; ++i) w16[i] = _cvtss_sh(wf[i], 0); /* f16, round to nearest even (F16C) */
    float *a1 = malloc(m * n * sizeof(float)), *a4 = malloc(m * n * sizeof(float));
    ora_linear_f16(p1, x, m, kk, w16, bias, n, a1);
    ora_linear_f16(p4, x, m, kk, w16, bias, n, a4);
    if (memcmp(a1, a4, m * n * sizeof(float))) { printf("FAIL linear f16: 1 vs 4 threads\n"); ++fails; }
    int8_t *q8 = malloc(n * kk);
    float *s8 = malloc(n * (kk / 32) * sizeof(float));
    ora_q8_quantize(wf, n, kk, q8, s8);
    ora_linear_q8(p1, x, m, kk, q8, s8, bias, n, a1);
    ora_linear_q8(p4, x, m, kk, q8, s8, bias, n, a4);
    if (memcmp(a1, a4, m * n * sizeof(float))) { printf("FAIL linear q8: 1 vs 4 threads\n"); ++fails; }
    float *lw = randv(kk), *lb = randv(kk), *y1 = malloc(m * kk * sizeof(float)), *y4 = malloc(m * kk * sizeof(float));
    ora_layer_norm(p1, x, m, kk, lw, lb, 1e-5f, y1);
    ora_layer_norm(p4, x, m, kk, lw, lb, 1e-5f, y4);
    if (memcmp(y1, y4, m * kk * sizeof(float))) { printf("FAIL layer norm: 1 vs 4 threads\n"); ++fails; }
    ora_gelu(p1, y1, m * kk);
    ora_gelu(p4, y4, m * kk);
    if (memcmp(y1, y4, m * kk * sizeof(float))) { printf("FAIL gelu: 1 vs 4 threads\n"); ++fails; }
    free(x), free(wf), free(bias), free(w16), free(a1), free(a4), free(q8), free(s8), free(lw), free(lb), free(y1), free(y4);

    ora_pool_free(p1);
    ora_pool_free(p4);
    printf("oracle: %d failures\n", fails);
    if (!fails) printf("ok\n");
    return fails ? 1 : 0;
}
