/*
 * refcpu.c -- CPU restatement of the odin-infer reference's CPU token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker.  The product library
 * (odin-infer_amd/csrc) never links, loads or calls it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the vajraimb/odin-infer tree).  The Odin toolchain is absent, so the
 * reference binary cannot be run; this restatement keeps the reference's
 * evaluation order:
 *   - dequant: separately rounded mul / mul / sub, no FMA (ggml/quant.odin:76-247)
 *   - dot_f32: two 8-lane FMA accumulators, ordered lane sum (ggml/quant.odin:250-269)
 *   - matmul_t: atomic per-row work queue over a thread pool, the caller
 *     participates, one dequant scratch per thread (infer/matmul.odin:28-109)
 *   - forward: infer/forward.odin:17-146
 * Built with -ffp-contract=off so the compiler adds no FMA of its own.
 *
 * Pinning (what checks each function; the tests live in tests/test_oracle.py):
 *   ref_f16_to_f32        all 65536 patterns vs numpy float16
 *   ref_get_scale_min_k4  exhaustive over all 8 j and 2^12-bit patterns vs an
 *                         independent bit-field model
 *   ref_dequant_row       independent element-wise forms (the reference's
 *                         k4_dequant_elem / k6_dequant_elem, qwen3_5/metal.odin:
 *                         476-486, 542-555) restated in numpy; closed-form KATs;
 *                         committed golden fixtures
 *   ref_dot_f32           float64 brute force; exact small-integer cases
 *   ref_matmul_t          float64 brute force; thread-count invariance
 *   ref_rmsnorm           KAT [3,4] -> x/sqrt(12.5) (qwen3_5/tests.odin:127-139)
 *   ref_softmax           closed form, float64
 *   ref_argmax            ties go to the lowest index (sampler/sampler.odin:79-89)
 *   forward               float64 re-computation of one layer on a tiny model;
 *                         position-0 attention identity; committed logits fixture
 *   ref_gemm_f16          batched prefill projection: all-ones / identity / row-
 *                         and column-distinct ladder (gemm_harness/gemm_test.odin
 *                         :1058-1067) with closed-form results; numpy float64
 *                         matmul of the f16-rounded dequantized rows
 * Bit-level equality with the Odin binary (its simd/libm lowering) stays
 * unpinned: parity is stated at tolerance level (1e-3) and greedy ids.
 */
#define _GNU_SOURCE
#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define EXPORT __attribute__((visibility("default")))

/* ggml type ids, ggml/gguf.odin:27-42 */
enum {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7,
    T_Q8_0 = 8, T_Q8_1 = 9, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12,
    T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15
};
#define QK_K 256

static char g_err[512];
EXPORT const char *ref_last_error(void) { return g_err; }

/* ---------------------------------------------------------------- quant --- */

/* ggml/quant.odin:10-42 */
EXPORT void ref_block_info(int k, int *elems, int *bytes) {
    int e = 1, b = 4;
    switch (k) {
    case T_F32: e = 1; b = 4; break;
    case T_F16: e = 1; b = 2; break;
    case T_Q4_0: e = 32; b = 18; break;
    case T_Q4_1: e = 32; b = 20; break;
    case T_Q5_0: e = 32; b = 22; break;
    case T_Q5_1: e = 32; b = 24; break;
    case T_Q8_0: e = 32; b = 34; break;
    case T_Q8_1: e = 32; b = 36; break;
    case T_Q2_K: e = 256; b = 84; break;
    case T_Q3_K: e = 256; b = 110; break;
    case T_Q4_K: e = 256; b = 144; break;
    case T_Q5_K: e = 256; b = 176; break;
    case T_Q6_K: e = 256; b = 210; break;
    case T_Q8_K: e = 256; b = 292; break;
    default: break;
    }
    *elems = e;
    *bytes = b;
}

/* ggml/quant.odin:44-47 */
EXPORT int64_t ref_row_byte_size(int k, int64_t n) {
    int e, b;
    ref_block_info(k, &e, &b);
    return (n / e) * b;
}

/* ggml/quant.odin:49-55 */
EXPORT int ref_is_supported_quant(int k) {
    switch (k) {
    case T_F32: case T_F16: case T_Q8_0: case T_Q4_0: case T_Q4_1:
    case T_Q5_0: case T_Q5_1: case T_Q4_K: case T_Q6_K:
        return 1;
    default:
        return 0;
    }
}

/* IEEE binary16 -> binary32, exact widening (ggml/quant.odin:58-61).
 * Written from the format definition: 1 sign, 5 exponent (bias 15), 10 mantissa. */
EXPORT float ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24, renormalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13); /* inf / nan, payload kept */
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float f16_at(const uint8_t *b) {
    return ref_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
}

/* binary32 -> binary16, round to nearest even (the f16 KV store of the
 * reference's GPU path rounds this way: infer/metal.odin:443-454). */
EXPORT uint16_t ref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0));
    if (ax >= 0x477FF000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* below 2^-14: subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); f16 unit 2^-24 */
        uint32_t q = m >> (shift - 0);
        /* q currently in units of 2^(e-150+shift) = 2^-24 */
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

/* ggml/quant.odin:64-73 */
EXPORT void ref_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ggml/quant.odin:178-209 */
static void dequant_q4_k(const uint8_t *src, int64_t n, float *dst) {
    int64_t nsb = n / QK_K;
    for (int64_t sb = 0; sb < nsb; sb++) {
        const uint8_t *base = src + sb * 144;
        float d = f16_at(base);
        float dmin = f16_at(base + 2);
        const uint8_t *scales = base + 4;
        const uint8_t *qs = base + 16;
        float *y = dst + sb * QK_K;
        int is = 0;
        for (int j = 0; j < QK_K; j += 64) {
            uint8_t sc0, m0, sc1, m1;
            ref_get_scale_min_k4(is + 0, scales, &sc0, &m0);
            ref_get_scale_min_k4(is + 1, scales, &sc1, &m1);
            float d1 = d * (float)sc0;
            float mm1 = dmin * (float)m0;
            float d2 = d * (float)sc1;
            float mm2 = dmin * (float)m1;
            for (int l = 0; l < 32; l++) y[l] = d1 * (float)(qs[l] & 0xF) - mm1;
            for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float)(qs[l] >> 4) - mm2;
            qs += 32;
            is += 2;
            y += 64;
        }
    }
}

/* ggml/quant.odin:212-247 */
static void dequant_q6_k(const uint8_t *src, int64_t n, float *dst) {
    int64_t nsb = n / QK_K;
    for (int64_t sb = 0; sb < nsb; sb++) {
        const uint8_t *base = src + sb * 210;
        const uint8_t *ql = base;
        const uint8_t *qh = base + 128;
        const int8_t *sc = (const int8_t *)(base + 192);
        float d = f16_at(base + 208);
        float *y = dst + sb * QK_K;
        for (int h = 0; h < 2; h++) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                /* d * f32(sc) * f32(q): left to right, two roundings */
                y[l] = d * (float)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            ql += 64;
            qh += 32;
            sc += 8;
            y += 128;
        }
    }
}

/* ggml/quant.odin:76-175 */
EXPORT void ref_dequant_row(int k, const uint8_t *src, int64_t n, float *dst) {
    switch (k) {
    case T_F32:
        memcpy(dst, src, (size_t)n * 4);
        break;
    case T_F16:
        for (int64_t i = 0; i < n; i++) dst[i] = f16_at(src + 2 * i);
        break;
    case T_Q8_0: {
        int64_t nb = n / 32;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = src + b * 34;
            float d = f16_at(base);
            for (int j = 0; j < 32; j++) dst[b * 32 + j] = d * (float)(int8_t)base[2 + j];
        }
        break;
    }
    case T_Q4_0: {
        int64_t nb = n / 32;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = src + b * 18;
            float d = f16_at(base);
            const uint8_t *qs = base + 2;
            for (int j = 0; j < 16; j++) {
                float x0 = (float)((int32_t)(qs[j] & 0xF) - 8);
                float x1 = (float)((int32_t)(qs[j] >> 4) - 8);
                dst[b * 32 + j] = x0 * d;
                dst[b * 32 + j + 16] = x1 * d;
            }
        }
        break;
    }
    case T_Q4_1: {
        int64_t nb = n / 32;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = src + b * 20;
            float d = f16_at(base);
            float m = f16_at(base + 2);
            const uint8_t *qs = base + 4;
            for (int j = 0; j < 16; j++) {
                dst[b * 32 + j] = (float)(qs[j] & 0xF) * d + m;
                dst[b * 32 + j + 16] = (float)(qs[j] >> 4) * d + m;
            }
        }
        break;
    }
    case T_Q5_0: {
        int64_t nb = n / 32;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = src + b * 22;
            float d = f16_at(base);
            uint32_t qh = (uint32_t)base[2] | (uint32_t)base[3] << 8 |
                          (uint32_t)base[4] << 16 | (uint32_t)base[5] << 24;
            const uint8_t *qs = base + 6;
            for (int j = 0; j < 16; j++) {
                uint8_t xh0 = (uint8_t)((qh >> j) << 4) & 0x10;
                uint8_t xh1 = (uint8_t)(qh >> (j + 12)) & 0x10;
                int32_t x0 = (int32_t)((qs[j] & 0xF) | xh0) - 16;
                int32_t x1 = (int32_t)((qs[j] >> 4) | xh1) - 16;
                dst[b * 32 + j] = (float)x0 * d;
                dst[b * 32 + j + 16] = (float)x1 * d;
            }
        }
        break;
    }
    case T_Q5_1: {
        int64_t nb = n / 32;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *base = src + b * 24;
            float d = f16_at(base);
            float m = f16_at(base + 2);
            uint32_t qh = (uint32_t)base[4] | (uint32_t)base[5] << 8 |
                          (uint32_t)base[6] << 16 | (uint32_t)base[7] << 24;
            const uint8_t *qs = base + 8;
            for (int j = 0; j < 16; j++) {
                uint8_t xh0 = (uint8_t)((qh >> j) << 4) & 0x10;
                uint8_t xh1 = (uint8_t)(qh >> (j + 12)) & 0x10;
                int32_t x0 = (int32_t)((qs[j] & 0xF) | xh0);
                int32_t x1 = (int32_t)((qs[j] >> 4) | xh1);
                dst[b * 32 + j] = (float)x0 * d + m;
                dst[b * 32 + j + 16] = (float)x1 * d + m;
            }
        }
        break;
    }
    case T_Q4_K:
        dequant_q4_k(src, n, dst);
        break;
    case T_Q6_K:
        dequant_q6_k(src, n, dst);
        break;
    default: /* Q8_1, Q2_K, Q3_K, Q5_K, Q8_K: zero-filled (quant.odin:170-173) */
        memset(dst, 0, (size_t)n * 4);
        break;
    }
}

/* Summation order of ref_dot_f32: 0 = the reference's (16-element steps from
 * the start of the row); 1 = the same steps taken from the end of the row.
 * Order 1 is a second, equally valid f32 evaluation of the same algorithm: the
 * tests use the difference of the two to measure how far f32 rounding alone
 * moves the oracle's logits (its "reordering noise") at a greedy near-tie. */
static volatile int g_dot_order;
EXPORT void ref_set_dot_order(int order) { g_dot_order = order; }

/* ggml/quant.odin:250-269: acc0/acc1 are 8-lane vectors updated with FMA over
 * 16-element steps; the lanes of acc0+acc1 are summed in order; scalar tail. */
EXPORT float ref_dot_f32(const float *a, const float *b, int64_t n) {
    float acc0[8] = {0}, acc1[8] = {0};
    int64_t i = 0;
    if (g_dot_order == 1) {
        for (int64_t j = (n / 16) * 16 - 16; j >= 0; j -= 16) {
            for (int k = 0; k < 8; k++) acc0[k] = fmaf(a[j + k], b[j + k], acc0[k]);
            for (int k = 0; k < 8; k++) acc1[k] = fmaf(a[j + 8 + k], b[j + 8 + k], acc1[k]);
        }
        i = (n / 16) * 16;
    }
    for (; g_dot_order != 1 && i + 16 <= n; i += 16) {
        for (int k = 0; k < 8; k++) acc0[k] = fmaf(a[i + k], b[i + k], acc0[k]);
        for (int k = 0; k < 8; k++) acc1[k] = fmaf(a[i + 8 + k], b[i + 8 + k], acc1[k]);
    }
    float s[8];
    for (int k = 0; k < 8; k++) s[k] = acc0[k] + acc1[k];
    float sum = s[0];
    for (int k = 1; k < 8; k++) sum = sum + s[k];
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* ggml/quant.odin:273-282 */
static float dot_row(int k, const uint8_t *src, const float *x, int64_t n, float *scratch) {
    if (k == T_F32) return ref_dot_f32((const float *)src, x, n);
    ref_dequant_row(k, src, n, scratch);
    return ref_dot_f32(scratch, x, n);
}

/* --------------------------------------------------------------- matmul --- */
/* infer/matmul.odin:10-109.  A persistent pool of (n-1) workers plus the
 * calling thread pull rows through one atomic counter; every row is computed
 * by exactly one thread, so results do not depend on the thread count. */

#define MAX_MATMUL_N 262144 /* per-thread scratch (qwen3_5/matmul.odin:10 size) */

typedef struct {
    int kind;
    const uint8_t *w;
    const float *x;
    float *xout;
    int64_t n, d, row_bytes;
    atomic_long next_row;
} mm_ctx;

typedef struct {
    int nthreads;
    pthread_t *th;
    float **scratch;
    pthread_mutex_t mu;
    pthread_cond_t cv;
    long generation;
    mm_ctx *job;
    atomic_int outstanding;
    int stop;
} mm_pool;

static void run_rows(mm_ctx *c, float *scratch) { /* infer/matmul.odin:63-70 */
    for (;;) {
        long row = atomic_fetch_add(&c->next_row, 1);
        if (row >= c->d) break;
        c->xout[row] = dot_row(c->kind, c->w + row * c->row_bytes, c->x, c->n, scratch);
    }
}

typedef struct { mm_pool *p; int idx; } worker_arg;

static void *worker_main(void *arg) {
    worker_arg *wa = (worker_arg *)arg;
    mm_pool *p = wa->p;
    int idx = wa->idx;
    free(wa);
    long seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        while (p->generation == seen && !p->stop) pthread_cond_wait(&p->cv, &p->mu);
        if (p->stop) { pthread_mutex_unlock(&p->mu); break; }
        seen = p->generation;
        mm_ctx *job = p->job;
        pthread_mutex_unlock(&p->mu);
        run_rows(job, p->scratch[idx]);
        atomic_fetch_sub(&p->outstanding, 1);
    }
    return NULL;
}

static mm_pool *pool_create(int nthreads) { /* infer/matmul.odin:32-46 */
    mm_pool *p = (mm_pool *)calloc(1, sizeof(mm_pool));
    p->nthreads = nthreads < 1 ? 1 : nthreads;
    p->scratch = (float **)calloc((size_t)p->nthreads, sizeof(float *));
    for (int i = 0; i < p->nthreads; i++) p->scratch[i] = (float *)malloc(MAX_MATMUL_N * sizeof(float));
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->cv, NULL);
    if (p->nthreads > 1) {
        p->th = (pthread_t *)calloc((size_t)p->nthreads - 1, sizeof(pthread_t));
        for (int i = 0; i < p->nthreads - 1; i++) {
            worker_arg *wa = (worker_arg *)malloc(sizeof(worker_arg));
            wa->p = p;
            wa->idx = i;
            pthread_create(&p->th[i], NULL, worker_main, wa);
        }
    }
    return p;
}

static void pool_destroy(mm_pool *p) { /* infer/matmul.odin:48-61 */
    if (!p) return;
    pthread_mutex_lock(&p->mu);
    p->stop = 1;
    pthread_cond_broadcast(&p->cv);
    pthread_mutex_unlock(&p->mu);
    for (int i = 0; i < p->nthreads - 1; i++) pthread_join(p->th[i], NULL);
    for (int i = 0; i < p->nthreads; i++) free(p->scratch[i]);
    free(p->scratch);
    free(p->th);
    free(p);
}

/* xout[d] = W[d,n] * x[n]  (infer/matmul.odin:77-109) */
static void matmul_t(mm_pool *p, float *xout, const float *x, int kind, const uint8_t *w,
                     int64_t n, int64_t d) {
    mm_ctx c;
    c.kind = kind;
    c.w = w;
    c.x = x;
    c.xout = xout;
    c.n = n;
    c.d = d;
    c.row_bytes = ref_row_byte_size(kind, n);
    atomic_init(&c.next_row, 0);
    if (p->nthreads <= 1) {
        run_rows(&c, p->scratch[0]);
        return;
    }
    atomic_store(&p->outstanding, p->nthreads - 1);
    pthread_mutex_lock(&p->mu);
    p->job = &c;
    p->generation++;
    pthread_cond_broadcast(&p->cv);
    pthread_mutex_unlock(&p->mu);
    run_rows(&c, p->scratch[p->nthreads - 1]); /* caller uses the last slot */
    while (atomic_load(&p->outstanding) > 0) sched_yield();
}

static mm_pool *g_pool;
static int g_pool_threads;

/* Standalone GEMV entry for the tests and the CPU microbench. */
EXPORT int ref_matmul_t(float *xout, const float *x, int kind, const uint8_t *w, int64_t n,
                        int64_t d, int nthreads) {
    if (n > MAX_MATMUL_N) {
        snprintf(g_err, sizeof g_err, "n=%lld exceeds MAX_MATMUL_N", (long long)n);
        return -1;
    }
    if (!g_pool || g_pool_threads != nthreads) {
        pool_destroy(g_pool);
        g_pool = pool_create(nthreads);
        g_pool_threads = nthreads;
    }
    matmul_t(g_pool, xout, x, kind, w, n, d);
    return 0;
}

EXPORT void ref_pool_shutdown(void) {
    pool_destroy(g_pool);
    g_pool = NULL;
    g_pool_threads = 0;
}

/* ------------------------------------------------------------------ ops --- */

/* infer/ops.odin:7-19 */
EXPORT void ref_rmsnorm(float *o, const float *x, const float *weight, int64_t size, float eps) {
    float ss = 0.0f;
    for (int64_t j = 0; j < size; j++) ss += x[j] * x[j];
    ss /= (float)size;
    ss += eps;
    ss = 1.0f / sqrtf(ss);
    for (int64_t j = 0; j < size; j++) o[j] = weight[j] * (ss * x[j]);
}

/* infer/ops.odin:21-37 */
EXPORT void ref_softmax(float *x, int64_t n) {
    if (n == 0) return;
    float max_val = x[0];
    for (int64_t i = 1; i < n; i++)
        if (x[i] > max_val) max_val = x[i];
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    for (int64_t i = 0; i < n; i++) x[i] /= sum;
}

/* sampler/sampler.odin:79-89: strict '>' so the lowest index wins ties */
EXPORT int64_t ref_argmax(const float *p, int64_t n) {
    int64_t max_i = 0;
    float max_p = p[0];
    for (int64_t i = 1; i < n; i++) {
        if (p[i] > max_p) {
            max_i = i;
            max_p = p[i];
        }
    }
    return max_i;
}

/* ----------------------------------------------------------------- gguf --- */
/* ggml/gguf.odin:9-229 */

enum { G_U8 = 0, G_I8, G_U16, G_I16, G_U32, G_I32, G_F32, G_BOOL, G_STR, G_ARR, G_U64, G_I64, G_F64 };

typedef struct {
    char key[96];
    int type;
    uint64_t u;
    double f;
    const char *str;
    uint64_t str_len;
} gmeta;

typedef struct {
    char name[96];
    int kind;
    int n_dims;
    uint64_t dims[4];
    uint64_t offset;
    const uint8_t *data;
    uint64_t size;
    uint8_t *copy; /* an aligned private copy when the file places data off 4-byte boundaries */
} gtensor;

typedef struct {
    uint8_t *map;
    size_t map_len;
    gmeta *meta;
    int n_meta;
    gtensor *tensors;
    int n_tensors;
} gfile;

typedef struct { const uint8_t *d; size_t len, pos; int bad; } rdr;

static int need(rdr *r, uint64_t n) {
    if (r->bad || n > r->len - r->pos) { r->bad = 1; return 0; } /* no wrap: pos <= len always */
    return 1;
}
static uint64_t rd_le(rdr *r, int n) {
    if (!need(r, (size_t)n)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)r->d[r->pos + i] << (8 * i);
    r->pos += (size_t)n;
    return v;
}
static const char *rd_str(rdr *r, uint64_t *len) {
    uint64_t l = rd_le(r, 8);
    if (!need(r, l)) return NULL;
    const char *s = (const char *)r->d + r->pos;
    r->pos += (size_t)l;
    *len = l;
    return s;
}
static void skip_val(rdr *r, int t, int depth) { /* gguf.odin:113-133 */
    if (depth > 4) { r->bad = 1; return; }
    uint64_t l;
    switch (t) {
    case G_U8: case G_I8: case G_BOOL: rd_le(r, 1); break;
    case G_U16: case G_I16: rd_le(r, 2); break;
    case G_U32: case G_I32: case G_F32: rd_le(r, 4); break;
    case G_U64: case G_I64: case G_F64: rd_le(r, 8); break;
    case G_STR: rd_str(r, &l); break;
    case G_ARR: {
        int et = (int)rd_le(r, 4);
        uint64_t c = rd_le(r, 8);
        for (uint64_t i = 0; i < c && !r->bad; i++) skip_val(r, et, depth + 1);
        break;
    }
    default: r->bad = 1; break;
    }
}

static void gfile_free(gfile *g) {
    if (g->map) munmap(g->map, g->map_len);
    for (int i = 0; g->tensors && i < g->n_tensors; i++) free(g->tensors[i].copy);
    free(g->meta);
    free(g->tensors);
    memset(g, 0, sizeof *g);
}

static int gfile_open(const char *path, gfile *g) { /* gguf.odin:167-229 */
    memset(g, 0, sizeof *g);
    int fd = open(path, O_RDONLY);
    if (fd < 0) { snprintf(g_err, sizeof g_err, "mmap failed for %s: %s", path, strerror(errno)); return -1; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        snprintf(g_err, sizeof g_err, "not a GGUF file (too short): %s", path);
        return -1;
    }
    g->map_len = (size_t)st.st_size;
    g->map = (uint8_t *)mmap(NULL, g->map_len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (g->map == MAP_FAILED) { g->map = NULL; snprintf(g_err, sizeof g_err, "mmap failed for %s", path); return -1; }
    rdr r = {g->map, g->map_len, 0, 0};
    uint32_t magic = (uint32_t)rd_le(&r, 4);
    if (magic != 0x46554747u) { snprintf(g_err, sizeof g_err, "not a GGUF file (magic=0x%x)", magic); return -2; }
    uint32_t version = (uint32_t)rd_le(&r, 4);
    if (version != 2 && version != 3) { snprintf(g_err, sizeof g_err, "unsupported GGUF version %u", version); return -3; }
    uint64_t tc = rd_le(&r, 8), mc = rd_le(&r, 8);
    if (tc > 1000000 || mc > 1000000) { snprintf(g_err, sizeof g_err, "corrupt GGUF header"); return -4; }
    g->meta = (gmeta *)calloc(mc ? mc : 1, sizeof(gmeta));
    for (uint64_t i = 0; i < mc && !r.bad; i++) {
        gmeta *m = &g->meta[g->n_meta++];
        uint64_t kl;
        const char *k = rd_str(&r, &kl);
        if (!k) break;
        snprintf(m->key, sizeof m->key, "%.*s", (int)(kl < sizeof m->key ? kl : sizeof m->key - 1), k);
        m->type = (int)rd_le(&r, 4);
        switch (m->type) { /* gguf.odin:135-161 */
        case G_U8: case G_I8: case G_BOOL: m->u = rd_le(&r, 1); break;
        case G_U16: case G_I16: m->u = rd_le(&r, 2); break;
        case G_U32: case G_I32: m->u = rd_le(&r, 4); break;
        case G_U64: case G_I64: m->u = rd_le(&r, 8); break;
        case G_F32: { uint32_t b = (uint32_t)rd_le(&r, 4); float f; memcpy(&f, &b, 4); m->f = f; break; }
        case G_F64: { uint64_t b = rd_le(&r, 8); memcpy(&m->f, &b, 8); break; }
        case G_STR: m->str = rd_str(&r, &m->str_len); break;
        case G_ARR: {
            int et = (int)rd_le(&r, 4);
            uint64_t c = rd_le(&r, 8);
            for (uint64_t j = 0; j < c && !r.bad; j++) skip_val(&r, et, 1);
            break;
        }
        default: r.bad = 1; break;
        }
    }
    g->tensors = (gtensor *)calloc(tc ? tc : 1, sizeof(gtensor));
    for (uint64_t i = 0; i < tc && !r.bad; i++) {
        gtensor *t = &g->tensors[g->n_tensors++];
        uint64_t nl;
        const char *nm = rd_str(&r, &nl);
        if (!nm) break;
        snprintf(t->name, sizeof t->name, "%.*s", (int)(nl < sizeof t->name ? nl : sizeof t->name - 1), nm);
        t->n_dims = (int)rd_le(&r, 4);
        if (t->n_dims < 1 || t->n_dims > 4) { r.bad = 1; break; }
        for (int d = 0; d < t->n_dims; d++) t->dims[d] = rd_le(&r, 8);
        t->kind = (int)rd_le(&r, 4);
        t->offset = rd_le(&r, 8);
    }
    if (r.bad) { snprintf(g_err, sizeof g_err, "truncated or corrupt GGUF"); return -5; }
    uint64_t alignment = 32;
    for (int i = 0; i < g->n_meta; i++)
        if (!strcmp(g->meta[i].key, "general.alignment")) alignment = g->meta[i].u;
    if (alignment == 0 || (alignment & (alignment - 1)) || alignment > g->map_len) { snprintf(g_err, sizeof g_err, "bad alignment"); return -6; }
    uint64_t data_base = (r.pos + alignment - 1) & ~(alignment - 1);
    for (int i = 0; i < g->n_tensors; i++) {
        gtensor *t = &g->tensors[i];
        /* element counts, sizes and offsets checked for wrap-around before use */
        uint64_t ne = 1;
        int e, b;
        ref_block_info(t->kind, &e, &b);
        for (int d = 0; d < t->n_dims; d++) {
            if (t->dims[d] && ne > (uint64_t)INT64_MAX / t->dims[d]) ne = UINT64_MAX;
            else ne *= t->dims[d];
        }
        if (ne == UINT64_MAX || ne / (uint64_t)e > (uint64_t)INT64_MAX / (uint64_t)b) {
            snprintf(g_err, sizeof g_err, "tensor %s: element count overflows", t->name);
            return -7;
        }
        if (t->offset % alignment) { /* spec placement; the reference does not check it */
            snprintf(g_err, sizeof g_err, "tensor %s is not aligned", t->name);
            return -7;
        }
        t->size = (uint64_t)ref_row_byte_size(t->kind, (int64_t)ne);
        if (t->offset > g->map_len || data_base > g->map_len - t->offset ||
            t->size > g->map_len - (data_base + t->offset)) {
            snprintf(g_err, sizeof g_err, "tensor %s extends past end of file", t->name);
            return -7;
        }
        t->data = g->map + data_base + t->offset;
        /* general.alignment 1 or 2 is legal GGUF but leaves f32/f16 data
         * misaligned for direct loads: read such a tensor from a copy */
        if (((uintptr_t)t->data & 3) && t->size) {
            t->copy = (uint8_t *)malloc((size_t)t->size);
            if (!t->copy) { snprintf(g_err, sizeof g_err, "out of memory"); return -7; }
            memcpy(t->copy, t->data, (size_t)t->size);
            t->data = t->copy;
        }
    }
    return 0;
}

static gmeta *gmeta_get(gfile *g, const char *k) {
    for (int i = 0; i < g->n_meta; i++)
        if (!strcmp(g->meta[i].key, k)) return &g->meta[i];
    return NULL;
}
static gtensor *gtensor_get(gfile *g, const char *k) {
    for (int i = 0; i < g->n_tensors; i++)
        if (!strcmp(g->tensors[i].name, k)) return &g->tensors[i];
    return NULL;
}

/* ---------------------------------------------------------------- model --- */
/* infer/model.odin:12-242 */

typedef struct { int kind; const uint8_t *data; } tensor;

typedef struct {
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
    tensor wq, wk, wv, wo, w1, w2, w3;
    /* layer kind: 0 Qwen3 attention (infer/forward.odin), 1 Qwen3.5 full attention,
     * 2 Qwen3.5 gated DeltaNet (qwen3_5/forward.odin:46-225) */
    int kind;
    /* routed-expert FFN (Qwen3-MoE / Qwen3-Next convention; no reference code),
     * optionally with a sigmoid-gated shared expert */
    int moe, shared;
    tensor router, gexp, uexp, dexp, sh_inp, sh_gate, sh_up, sh_down;
    /* gated DeltaNet (qwen3_5/model.odin:346-360) and its states */
    tensor in_qkv, in_z, in_b, in_a, ssm_out;
    const float *conv_w, *dt_bias, *ssm_a, *ssm_norm;
    float *conv_state, *rec_state;
    /* Qwen3.5 full attention: f16 cache [n_kv][seq_len][head_dim] (binary16 bits) */
    uint16_t *kc16, *vc16;
} layer_w;

typedef struct {
    /* Config, field order of infer/model.odin:12-24 */
    int64_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, max_seq, head_dim;
    float rope_freq, rms_eps;
    tensor token_embedding, output;
    const float *output_norm;
    layer_w *layers;
    /* architecture: 0 "qwen3" (infer/model.odin), 1 "qwen3moe", 2 "qwen35" (qwen3_5/model.odin) */
    int arch;
    int64_t n_experts, top_k, expert_ffn, shared_ffn;
    int norm_topk;
    int64_t rotary_dim, lin_nk, lin_nv, lin_hk, lin_hv, lin_kernel, full_interval;
    float *inv_freq;
    /* scratch of the MoE and hybrid layers */
    float *mo_p, *mo_h, *mo_y, *mo_t, *hy_qproj, *hy_k, *hy_v, *hy_qkv, *hy_z, *hy_b, *hy_a, *hy_out;
    /* Run_State, infer/model.odin:53-65 */
    float *x, *xb, *xb2, *xb3, *hb, *hb2, *q, *att, *logits, *key_cache, *value_cache;
    float *ktmp, *vtmp;
    int kv_f16;
    gfile g;
    mm_pool *pool;
    /* f16-rounded dequantized projection weights of the batched path, per
     * tensor, made on first use (ref_engine_prefill) */
    const uint8_t **stg_key;
    float **stg_w;
    int n_stg;
    /* engine_verify_batch: logits of every position [vf_rows][vocab] */
    float *vf;
    int64_t vf_rows;
    /* test hook: the routing boundary of every (position, layer) a forward
     * visits, log(p_k / p_k+1) of the k-th chosen and the best unchosen
     * expert, [seq_len][n_layers] (NAN where no routed FFN ran) */
    float *rt_margin;
    int64_t cur_pos, cur_layer;
} ref_engine;

static float ref_sigmoid(float x);
static float ref_silu(float x);
EXPORT void ref_inv_freq(float theta, int rotary_dim, float *out);
EXPORT int ref_deltanet_steps(int n_kh, int n_vh, int hk, int hv, int kernel, float eps, int n_tokens,
                              const float *qkv, const float *z, const float *b, const float *a, const float *conv_w,
                              const float *a_decay, const float *dt_bias, const float *norm_w, float *conv_state,
                              float *rec_state, float *out);
EXPORT int ref_qwen35_attn_steps(int n_heads, int n_kv, int hd, int rotary_dim, int seq_len, float eps, int n_tokens,
                                 int pos0, const float *qproj, const float *k, const float *v, const float *q_norm,
                                 const float *k_norm, const float *inv_freq, uint16_t *kc, uint16_t *vc, float *out);

static int require(ref_engine *e, const char *name, gtensor **out) { /* infer/model.odin:82-97 */
    gtensor *t = gtensor_get(&e->g, name);
    if (!t) { snprintf(g_err, sizeof g_err, "missing required tensor: %s", name); return -10; }
    if (!ref_is_supported_quant(t->kind)) {
        snprintf(g_err, sizeof g_err, "tensor %s has unsupported quant type %d", name, t->kind);
        return -11;
    }
    *out = t;
    return 0;
}

static int as_f32(ref_engine *e, const char *name, const float **out) { /* infer/model.odin:74-80 */
    gtensor *t;
    int rc = require(e, name, &t);
    if (rc) return rc;
    if (t->kind != T_F32) { snprintf(g_err, sizeof g_err, "expected F32 tensor for %s", name); return -12; }
    *out = (const float *)t->data;
    return 0;
}

/* Shape checks the reference leaves to Odin's bounds-checked slices: a
 * weight's rows hold `cols` elements and it has `rows` of them (3-D expert
 * stacks count every expert's rows), so the forward pass never reads past a
 * tensor.  Not a reference step; malformed files fail here instead. */
static int shape_ok(ref_engine *e, const gtensor *t, int64_t cols, int64_t rows) {
    uint64_t ne = 1;
    for (int d = 0; d < t->n_dims; d++) ne *= t->dims[d]; /* bounded by the reader's overflow check */
    if (t->dims[0] != (uint64_t)cols || ne != (uint64_t)cols * (uint64_t)rows) {
        snprintf(g_err, sizeof g_err, "tensor %s: shape does not match the model's dimensions", t->name);
        (void)e;
        return 0;
    }
    return 1;
}

EXPORT void ref_engine_destroy(void *h) {
    ref_engine *e = (ref_engine *)h;
    if (!e) return;
    free(e->x); free(e->xb); free(e->xb2); free(e->xb3); free(e->hb); free(e->hb2);
    free(e->q); free(e->att); free(e->logits); free(e->key_cache); free(e->value_cache);
    free(e->ktmp); free(e->vtmp);
    free(e->inv_freq); free(e->mo_p); free(e->mo_h); free(e->mo_y); free(e->mo_t);
    free(e->hy_qproj); free(e->hy_k); free(e->hy_v); free(e->hy_qkv); free(e->hy_z); free(e->hy_b);
    free(e->hy_a); free(e->hy_out);
    for (int64_t l = 0; e->layers && l < e->n_layers; l++) {
        free(e->layers[l].conv_state); free(e->layers[l].rec_state);
        free(e->layers[l].kc16); free(e->layers[l].vc16);
    }
    for (int i = 0; i < e->n_stg; i++) free(e->stg_w[i]);
    free(e->stg_key); free(e->stg_w);
    free(e->vf);
    free(e->rt_margin);
    free(e->layers);
    pool_destroy(e->pool);
    gfile_free(&e->g);
    free(e);
}

/* engine_load (infer/engine.odin:18-34) -> build_transformer (infer/model.odin:216-242).
 * kv_f16 != 0 selects the f16 KV mode: K and V at each position are rounded to
 * binary16 (round-to-nearest-even) when stored, as the reference GPU path's
 * store_kv does (infer/metal.odin:443-454), and attention reads them back. */
EXPORT void *ref_engine_load(const char *path, int max_ctx, int num_threads, int kv_f16) {
    ref_engine *e = (ref_engine *)calloc(1, sizeof(ref_engine));
    int rc = gfile_open(path, &e->g);
    if (rc) { ref_engine_destroy(e); return NULL; }
    gfile *g = &e->g;
    /* load_config (infer/model.odin:99-139; qwen3_5/model.odin:225-304): the
     * metadata keys carry the architecture name as their prefix */
    gmeta *am = gmeta_get(g, "general.architecture");
    char arch[32] = "qwen3";
    if (am && am->str && am->str_len < sizeof arch) {
        memcpy(arch, am->str, am->str_len);
        arch[am->str_len] = 0;
    }
    e->arch = !strcmp(arch, "qwen3moe") ? 1 : !strcmp(arch, "qwen35") ? 2 : 0;
    char key[128];
#define META_U(dst, suffix) do { snprintf(key, sizeof key, "%s." suffix, arch); gmeta *m_ = gmeta_get(g, key); \
        if (!m_) { snprintf(g_err, sizeof g_err, "missing metadata key: %s", key); ref_engine_destroy(e); return NULL; } \
        dst = (int64_t)m_->u; } while (0)
    META_U(e->dim, "embedding_length");
    META_U(e->hidden_dim, "feed_forward_length");
    META_U(e->n_layers, "block_count");
    META_U(e->n_heads, "attention.head_count");
    META_U(e->n_kv_heads, "attention.head_count_kv");
    META_U(e->max_seq, "context_length");
    META_U(e->head_dim, "attention.key_length");
    if (e->arch == 1 || (e->arch == 2 && (snprintf(key, sizeof key, "%s.expert_count", arch), gmeta_get(g, key)))) {
        META_U(e->n_experts, "expert_count");
        META_U(e->top_k, "expert_used_count");
        META_U(e->expert_ffn, "expert_feed_forward_length");
        e->hidden_dim = e->expert_ffn;
        e->norm_topk = 1; /* Qwen3-MoE / Qwen3-Next renormalize the chosen weights */
        snprintf(key, sizeof key, "%s.expert_shared_feed_forward_length", arch);
        gmeta *sm = gmeta_get(g, key);
        e->shared_ffn = sm ? (int64_t)sm->u : 0;
    }
    if (e->arch == 2) { /* qwen3_5/model.odin:262-300 */
        META_U(e->lin_nk, "ssm.group_count");
        META_U(e->lin_nv, "ssm.time_step_rank");
        META_U(e->lin_hk, "ssm.state_size");
        int64_t inner;
        META_U(inner, "ssm.inner_size");
        e->lin_hv = inner / (e->lin_nv > 0 ? e->lin_nv : 1);
        META_U(e->lin_kernel, "ssm.conv_kernel");
        META_U(e->full_interval, "full_attention_interval");
        META_U(e->rotary_dim, "rope.dimension_count");
    }
#undef META_U
    snprintf(key, sizeof key, "%s.rope.freq_base", arch);
    gmeta *m = gmeta_get(g, key);
    e->rope_freq = m ? (float)m->f : (e->arch == 2 ? 10000000.0f : 1000000.0f);
    snprintf(key, sizeof key, "%s.attention.layer_norm_rms_epsilon", arch);
    m = gmeta_get(g, key);
    e->rms_eps = m ? (float)m->f : 1e-6f;
    /* dimensions in range before anything is sized by them (not a reference
     * step: the reference trusts the file) */
    {
        const int64_t lim = 1 << 20;
        int ok = e->dim > 0 && e->dim <= lim && e->hidden_dim > 0 && e->hidden_dim <= lim && e->n_layers > 0 &&
                 e->n_layers <= 4096 && e->n_heads > 0 && e->n_heads <= 4096 && e->n_kv_heads > 0 &&
                 e->n_heads % e->n_kv_heads == 0 && e->head_dim > 0 && e->head_dim <= 4096 && max_ctx > 0;
        if (e->n_experts > 0 || e->arch == 1)
            ok = ok && e->n_experts > 0 && e->n_experts <= 4096 && e->top_k > 0 && e->top_k <= e->n_experts &&
                 e->expert_ffn > 0 && e->expert_ffn <= lim && e->shared_ffn >= 0 && e->shared_ffn <= lim;
        if (e->arch == 2)
            ok = ok && e->lin_nk > 0 && e->lin_nk <= 4096 && e->lin_nv > 0 && e->lin_nv <= 4096 && e->lin_hk > 0 &&
                 e->lin_hk <= 4096 && e->lin_hv > 0 && e->lin_hv <= 4096 && e->lin_kernel > 0 && e->lin_kernel <= 64 &&
                 e->full_interval > 0 && e->rotary_dim >= 0 && e->rotary_dim <= e->head_dim && e->rotary_dim % 2 == 0;
        if (!ok) {
            snprintf(g_err, sizeof g_err, "model dimensions out of range");
            ref_engine_destroy(e);
            return NULL;
        }
    }
    gtensor *emb;
    if (require(e, "token_embd.weight", &emb)) { ref_engine_destroy(e); return NULL; }
    e->vocab_size = (int64_t)emb->dims[emb->n_dims - 1];
    if (e->vocab_size <= 0 || e->vocab_size > (1 << 24) || !shape_ok(e, emb, e->dim, e->vocab_size)) {
        if (e->vocab_size <= 0 || e->vocab_size > (1 << 24))
            snprintf(g_err, sizeof g_err, "vocabulary size out of range");
        ref_engine_destroy(e);
        return NULL;
    }
    /* infer/model.odin:220-223 */
    e->seq_len = e->max_seq < max_ctx ? e->max_seq : max_ctx;
    if (e->seq_len <= 0) e->seq_len = max_ctx;
    /* memory_map_weights, infer/model.odin:141-179 */
    e->token_embedding = (tensor){emb->kind, emb->data};
    if (as_f32(e, "output_norm.weight", &e->output_norm) || !shape_ok(e, gtensor_get(g, "output_norm.weight"), e->dim, 1)) {
        ref_engine_destroy(e);
        return NULL;
    }
    gtensor *out = gtensor_get(g, "output.weight");
    if (out) {
        if (!ref_is_supported_quant(out->kind)) {
            snprintf(g_err, sizeof g_err, "output.weight has unsupported quant type %d", out->kind);
            ref_engine_destroy(e);
            return NULL;
        }
        if (!shape_ok(e, out, e->dim, e->vocab_size)) { ref_engine_destroy(e); return NULL; }
        e->output = (tensor){out->kind, out->data};
    } else {
        e->output = e->token_embedding; /* tied classifier */
    }
    e->layers = (layer_w *)calloc((size_t)e->n_layers, sizeof(layer_w));
    if (!e->layers) { snprintf(g_err, sizeof g_err, "out of memory"); ref_engine_destroy(e); return NULL; }
    char nm[96];
    const int64_t conv_dim = 2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv;
    const int64_t D = e->dim, QD = e->n_heads * e->head_dim, KVD = e->n_kv_heads * e->head_dim;
    const int64_t VD = e->lin_nv * e->lin_hv, HD = e->head_dim;
    for (int64_t l = 0; l < e->n_layers; l++) {
        layer_w *lw = &e->layers[l];
        int bad = 0;
#define F32W(field, suffix, n) { snprintf(nm, sizeof nm, "blk.%lld." suffix, (long long)l); \
        if (as_f32(e, nm, &lw->field) || !shape_ok(e, gtensor_get(g, nm), n, 1)) bad = 1; }
#define QW(field, suffix, cols, rows) { gtensor *t_; snprintf(nm, sizeof nm, "blk.%lld." suffix, (long long)l); \
        if (require(e, nm, &t_) || !shape_ok(e, t_, cols, rows)) bad = 1; else lw->field = (tensor){t_->kind, t_->data}; }
        F32W(attn_norm, "attn_norm.weight", D)
        if (e->arch == 2) { F32W(ffn_norm, "post_attention_norm.weight", D) } /* qwen3_5/model.odin:325 */
        else { F32W(ffn_norm, "ffn_norm.weight", D) }
        lw->kind = e->arch != 2 ? 0 : ((l + 1) % e->full_interval == 0 ? 1 : 2); /* qwen3_5/model.odin:289-300 */
        if (lw->kind != 2) {
            F32W(q_norm, "attn_q_norm.weight", HD)
            F32W(k_norm, "attn_k_norm.weight", HD)
            QW(wq, "attn_q.weight", D, lw->kind == 1 ? 2 * QD : QD)
            QW(wk, "attn_k.weight", D, KVD)
            QW(wv, "attn_v.weight", D, KVD)
            QW(wo, "attn_output.weight", QD, D)
        } else {
            QW(in_qkv, "attn_qkv.weight", D, conv_dim)
            QW(in_z, "attn_gate.weight", D, VD)
            QW(in_b, "ssm_beta.weight", D, e->lin_nv)
            QW(in_a, "ssm_alpha.weight", D, e->lin_nv)
            { /* [conv_dim][kernel] F32 */
                snprintf(nm, sizeof nm, "blk.%lld.ssm_conv1d.weight", (long long)l);
                if (as_f32(e, nm, &lw->conv_w) || !shape_ok(e, gtensor_get(g, nm), e->lin_kernel, conv_dim)) bad = 1;
            }
            F32W(dt_bias, "ssm_dt.bias", e->lin_nv)
            F32W(ssm_a, "ssm_a", e->lin_nv)
            F32W(ssm_norm, "ssm_norm.weight", e->lin_hv)
            QW(ssm_out, "ssm_out.weight", VD, D)
        }
        if (e->n_experts > 0) {
            lw->moe = 1;
            QW(router, "ffn_gate_inp.weight", D, e->n_experts)
            QW(gexp, "ffn_gate_exps.weight", D, e->n_experts * e->expert_ffn)
            QW(uexp, "ffn_up_exps.weight", D, e->n_experts * e->expert_ffn)
            QW(dexp, "ffn_down_exps.weight", e->expert_ffn, e->n_experts * D)
            snprintf(nm, sizeof nm, "blk.%lld.ffn_gate_inp_shexp.weight", (long long)l);
            if (gtensor_get(g, nm)) {
                lw->shared = 1;
                if (e->shared_ffn <= 0) bad = 1;
                QW(sh_inp, "ffn_gate_inp_shexp.weight", D, 1)
                QW(sh_gate, "ffn_gate_shexp.weight", D, e->shared_ffn)
                QW(sh_up, "ffn_up_shexp.weight", D, e->shared_ffn)
                QW(sh_down, "ffn_down_shexp.weight", e->shared_ffn, D)
            }
        } else {
            QW(w1, "ffn_gate.weight", D, e->hidden_dim)
            QW(w2, "ffn_down.weight", e->hidden_dim, D)
            QW(w3, "ffn_up.weight", D, e->hidden_dim)
        }
#undef F32W
#undef QW
        if (bad) { ref_engine_destroy(e); return NULL; }
        if (lw->kind == 2) {
            lw->conv_state = (float *)calloc((size_t)(conv_dim * (e->lin_kernel - 1) + 1), 4);
            lw->rec_state = (float *)calloc((size_t)(e->lin_nv * e->lin_hk * e->lin_hv), 4);
        } else if (lw->kind == 1) {
            lw->kc16 = (uint16_t *)calloc((size_t)(e->n_kv_heads * e->seq_len * e->head_dim), 2);
            lw->vc16 = (uint16_t *)calloc((size_t)(e->n_kv_heads * e->seq_len * e->head_dim), 2);
        }
    }
    if (e->arch == 2) {
        e->inv_freq = (float *)calloc((size_t)(e->rotary_dim / 2 + 1), 4);
        ref_inv_freq(e->rope_freq, (int)e->rotary_dim, e->inv_freq); /* qwen3_5/model.odin:454-455 */
        e->hy_qproj = (float *)calloc((size_t)(2 * e->n_heads * e->head_dim), 4);
        e->hy_k = (float *)calloc((size_t)(e->n_kv_heads * e->head_dim), 4);
        e->hy_v = (float *)calloc((size_t)(e->n_kv_heads * e->head_dim), 4);
        e->hy_qkv = (float *)calloc((size_t)(conv_dim + 1), 4);
        e->hy_z = (float *)calloc((size_t)(e->lin_nv * e->lin_hv + 1), 4);
        e->hy_b = (float *)calloc((size_t)(e->lin_nv + 1), 4);
        e->hy_a = (float *)calloc((size_t)(e->lin_nv + 1), 4);
        e->hy_out = (float *)calloc((size_t)(e->lin_nv * e->lin_hv + e->n_heads * e->head_dim + 1), 4);
    }
    if (e->n_experts > 0) {
        int64_t hmax = e->expert_ffn > e->shared_ffn ? e->expert_ffn : e->shared_ffn;
        e->mo_p = (float *)calloc((size_t)e->n_experts, 4);
        e->mo_h = (float *)calloc((size_t)(e->top_k * hmax + 2 * hmax), 4);
        e->mo_y = (float *)calloc((size_t)e->dim, 4);
        e->mo_t = (float *)calloc((size_t)e->dim, 4);
    }
    /* malloc_run_state, infer/model.odin:185-200 */
    int64_t att_head_dim = e->n_heads * e->head_dim, kv_dim = e->n_kv_heads * e->head_dim;
    e->x = (float *)calloc((size_t)e->dim, 4);
    e->xb = (float *)calloc((size_t)e->dim, 4);
    e->xb2 = (float *)calloc((size_t)e->dim, 4);
    e->xb3 = (float *)calloc((size_t)att_head_dim, 4);
    e->hb = (float *)calloc((size_t)e->hidden_dim, 4);
    e->hb2 = (float *)calloc((size_t)e->hidden_dim, 4);
    e->q = (float *)calloc((size_t)att_head_dim, 4);
    e->att = (float *)calloc((size_t)(e->n_heads * e->seq_len), 4);
    e->logits = (float *)calloc((size_t)e->vocab_size, 4);
    e->key_cache = (float *)calloc((size_t)(e->n_layers * e->seq_len * kv_dim), 4);
    e->value_cache = (float *)calloc((size_t)(e->n_layers * e->seq_len * kv_dim), 4);
    e->ktmp = (float *)calloc((size_t)kv_dim, 4);
    e->vtmp = (float *)calloc((size_t)kv_dim, 4);
    if (!e->key_cache || !e->value_cache) { snprintf(g_err, sizeof g_err, "KV cache allocation failed"); ref_engine_destroy(e); return NULL; }
    {
        int missing = !e->x || !e->xb || !e->xb2 || !e->xb3 || !e->hb || !e->hb2 || !e->q || !e->att || !e->logits ||
                      !e->ktmp || !e->vtmp;
        if (e->arch == 2)
            missing |= !e->inv_freq || !e->hy_qproj || !e->hy_k || !e->hy_v || !e->hy_qkv || !e->hy_z || !e->hy_b ||
                       !e->hy_a || !e->hy_out;
        if (e->n_experts > 0) missing |= !e->mo_p || !e->mo_h || !e->mo_y || !e->mo_t;
        for (int64_t l = 0; l < e->n_layers; l++) {
            const layer_w *lw = &e->layers[l];
            if (lw->kind == 2) missing |= !lw->conv_state || !lw->rec_state;
            if (lw->kind == 1) missing |= !lw->kc16 || !lw->vc16;
        }
        if (missing) { snprintf(g_err, sizeof g_err, "out of memory"); ref_engine_destroy(e); return NULL; }
    }
    e->kv_f16 = kv_f16;
    e->pool = pool_create(num_threads < 1 ? 1 : num_threads); /* infer/engine.odin:20 */
    return e;
}

/* Config fields in infer/model.odin:12-24 order; floats returned as doubles. */
EXPORT void ref_engine_config(void *h, int64_t *ints9, float *floats2) {
    ref_engine *e = (ref_engine *)h;
    int64_t v[9] = {e->dim, e->hidden_dim, e->n_layers, e->n_heads, e->n_kv_heads,
                    e->vocab_size, e->seq_len, e->max_seq, e->head_dim};
    memcpy(ints9, v, sizeof v);
    floats2[0] = e->rope_freq;
    floats2[1] = e->rms_eps;
}

/* Overwrite positions [pos0, pos0+npos) of one layer's K and V with given
 * binary16 values laid out [kv_head][npos][head_dim]. */
EXPORT int ref_engine_kv_fill(void *h, int layer, int pos0, int npos, const uint16_t *k16, const uint16_t *v16) {
    ref_engine *e = (ref_engine *)h;
    if (layer < 0 || layer >= e->n_layers || pos0 < 0 || npos < 0 || pos0 + npos > e->seq_len) {
        snprintf(g_err, sizeof g_err, "kv_fill out of range");
        return -1;
    }
    int64_t kv_dim = e->n_kv_heads * e->head_dim, hd = e->head_dim;
    int64_t loff = (int64_t)layer * e->seq_len * kv_dim;
    for (int64_t kh = 0; kh < e->n_kv_heads; kh++)
        for (int64_t t = 0; t < npos; t++)
            for (int64_t i = 0; i < hd; i++) {
                int64_t src = (kh * npos + t) * hd + i;
                int64_t dst = loff + (pos0 + t) * kv_dim + kh * hd + i;
                e->key_cache[dst] = ref_f16_to_f32(k16[src]);
                e->value_cache[dst] = ref_f16_to_f32(v16[src]);
            }
    return 0;
}

/* The projection of the batched prefill path (forward_gpu_batch's MMQ,
 * qwen3_5/metal.odin:1236-1243, 493-609): weights dequantized and rounded to
 * f16, the input rounded to f16, products summed (in float64 here, as
 * ref_gemm_f16).  xout[d] = W[d][n] x[n]. */
static const float *staged_weights(ref_engine *e, int kind, const uint8_t *w, int64_t n, int64_t d) {
    for (int i = 0; i < e->n_stg; i++)
        if (e->stg_key[i] == w) return e->stg_w[i];
    float *sw = malloc((size_t)(n * d) * sizeof(float));
    const uint8_t **nk = realloc(e->stg_key, (size_t)(e->n_stg + 1) * sizeof *nk);
    float **nw = realloc(e->stg_w, (size_t)(e->n_stg + 1) * sizeof *nw);
    if (nk) e->stg_key = nk;
    if (nw) e->stg_w = nw;
    if (!sw || !nk || !nw) { free(sw); return NULL; }
    const int64_t rb = ref_row_byte_size(kind, n);
    for (int64_t r = 0; r < d; r++) {
        ref_dequant_row(kind, w + r * rb, n, sw + r * n);
        for (int64_t j = 0; j < n; j++) sw[r * n + j] = ref_f16_to_f32(ref_f32_to_f16(sw[r * n + j]));
    }
    e->stg_key[e->n_stg] = w;
    e->stg_w[e->n_stg++] = sw;
    return sw;
}

static int matmul_staged(ref_engine *e, float *xout, const float *x, int kind, const uint8_t *w, int64_t n,
                         int64_t d) {
    const float *sw = staged_weights(e, kind, w, n, d);
    double *xs = malloc((size_t)n * sizeof(double));
    if (!sw || !xs) {
        free(xs);
        snprintf(g_err, sizeof g_err, "prefill: out of memory");
        return -1;
    }
    for (int64_t j = 0; j < n; j++) xs[j] = ref_f16_to_f32(ref_f32_to_f16(x[j]));
    for (int64_t r = 0; r < d; r++) {
        double acc = 0.0;
        for (int64_t j = 0; j < n; j++) acc += (double)sw[r * n + j] * xs[j];
        xout[r] = (float)acc;
    }
    free(xs);
    return 0;
}

/* forward (infer/forward.odin:17-146); with `staged` the seven projections of
 * each layer are the batched path's (matmul_staged), and without `logits` the
 * final norm and classifier are skipped (forward_gpu_batch computes them for
 * the last token only, qwen3_5/metal.odin:1637-1641). */
/* Routed-expert SwiGLU FFN of one token (x already normalized) into y, rows on
 * the row pool: the arithmetic of ref_moe_ffn (each row dequantized and dotted
 * with dot_f32; softmax; top_k by a strict '>' scan, ties to the lower id;
 * weights renormalized in selection order; y[r] = sum over the chosen experts
 * in selection order of w_k * (down_e h_k)[r], h_k = silu(gate_e x) *
 * up_e x), then the shared expert when the layer has one (HF Qwen3-Next):
 * y += sigmoid(w_shexp . x) * down_s(silu(gate_s x) * up_s x).  The reference
 * has no MoE code (qwen3_5/model.odin:80-82 is a dense MLP). */
static void moe_ffn_layer(ref_engine *e, const layer_w *lw, const float *x, float *y) {
    const int64_t D = e->dim, E = e->n_experts, K = e->top_k, F = e->expert_ffn, S = e->shared_ffn;
    mm_pool *P = e->pool;
    float *p = e->mo_p, *h = e->mo_h, *t = e->mo_t;
    matmul_t(P, p, x, lw->router.kind, lw->router.data, D, E);
    ref_softmax(p, E);
    int ids[64];
    float w[64], sum = 0.0f;
    for (int64_t k = 0; k < K; k++) {
        int best = -1;
        for (int64_t i = 0; i < E; i++)
            if (p[i] >= 0.0f && (best < 0 || p[i] > p[best])) best = (int)i;
        if (best < 0) { /* NaN probabilities rank nothing: expert 0 at weight 0, as the device does */
            ids[k] = 0;
            w[k] = 0.0f;
            continue;
        }
        ids[k] = best;
        w[k] = p[best];
        sum += p[best];
        p[best] = -1.0f;
    }
    if (e->rt_margin && K > 0) {
        float nxt = -1.0f;
        for (int64_t i = 0; i < E; i++)
            if (p[i] > nxt) nxt = p[i];
        e->rt_margin[e->cur_pos * e->n_layers + e->cur_layer] = nxt > 0.0f ? logf(w[K - 1] / nxt) : INFINITY;
    }
    for (int64_t k = 0; k < K; k++) w[k] = e->norm_topk ? w[k] / sum : w[k];
    const int64_t grb = ref_row_byte_size(lw->gexp.kind, D), drb = ref_row_byte_size(lw->dexp.kind, F);
    float *hk = h, *hu = h + K * F;
    for (int64_t k = 0; k < K; k++) {
        const int64_t ex = ids[k];
        matmul_t(P, hk + k * F, x, lw->gexp.kind, lw->gexp.data + ex * F * grb, D, F);
        matmul_t(P, hu, x, lw->uexp.kind, lw->uexp.data + ex * F * grb, D, F);
        for (int64_t r = 0; r < F; r++) hk[k * F + r] = ref_silu(hk[k * F + r]) * hu[r];
    }
    for (int64_t r = 0; r < D; r++) y[r] = 0.0f;
    for (int64_t k = 0; k < K; k++) {
        matmul_t(P, t, hk + k * F, lw->dexp.kind, lw->dexp.data + (int64_t)ids[k] * D * drb, F, D);
        for (int64_t r = 0; r < D; r++) y[r] += w[k] * t[r];
    }
    if (!lw->shared) return;
    float g;
    matmul_t(P, &g, x, lw->sh_inp.kind, lw->sh_inp.data, D, 1);
    float *sg = h, *su = h + S;
    matmul_t(P, sg, x, lw->sh_gate.kind, lw->sh_gate.data, D, S);
    matmul_t(P, su, x, lw->sh_up.kind, lw->sh_up.data, D, S);
    for (int64_t r = 0; r < S; r++) sg[r] = ref_silu(sg[r]) * su[r];
    matmul_t(P, t, sg, lw->sh_down.kind, lw->sh_down.data, S, D);
    const float gs = ref_sigmoid(g);
    for (int64_t r = 0; r < D; r++) y[r] += gs * t[r];
}

/* a projection of the per-token path (matmul_t) or, with `staged`, of the
 * batched path (matmul_staged) */
static int matmul_mode(ref_engine *e, int staged, float *out, const float *in, const tensor *t, int64_t n,
                       int64_t d) {
    if (!staged) {
        matmul_t(e->pool, out, in, t->kind, t->data, n, d);
        return 0;
    }
    return matmul_staged(e, out, in, t->kind, t->data, n, d);
}

/* forward_full_layer (qwen3_5/forward.odin:46-135) up to the residual add:
 * RMSNorm, the [q | gate], k and v projections, then the attention restated by
 * ref_qwen35_attn_steps (q/k RMSNorm, partial RoPE, f16 cache at pos, softmax
 * with dot * 1/sqrt(head_dim), sigmoid gate), wo. */
static int q35_full_attention(ref_engine *e, layer_w *lw, int pos, int staged) {
    const int64_t D = e->dim, QD = e->n_heads * e->head_dim, KVD = e->n_kv_heads * e->head_dim;
    ref_rmsnorm(e->xb, e->x, lw->attn_norm, D, e->rms_eps);
    if (matmul_mode(e, staged, e->hy_qproj, e->xb, &lw->wq, D, 2 * QD) ||
        matmul_mode(e, staged, e->hy_k, e->xb, &lw->wk, D, KVD) ||
        matmul_mode(e, staged, e->hy_v, e->xb, &lw->wv, D, KVD))
        return -1;
    if (ref_qwen35_attn_steps((int)e->n_heads, (int)e->n_kv_heads, (int)e->head_dim, (int)e->rotary_dim,
                              (int)e->seq_len, e->rms_eps, 1, pos, e->hy_qproj, e->hy_k, e->hy_v, lw->q_norm,
                              lw->k_norm, e->inv_freq, lw->kc16, lw->vc16, e->hy_out))
        return -1;
    if (matmul_mode(e, staged, e->xb2, e->hy_out, &lw->wo, QD, D)) return -1;
    for (int64_t i = 0; i < D; i++) e->x[i] += e->xb2[i];
    return 0;
}

/* forward_linear_layer (qwen3_5/forward.odin:137-225) up to the residual add:
 * RMSNorm, the in_qkv / in_z / in_b / in_a projections, the conv / l2norm /
 * delta rule / gated RMSNorm step restated by ref_deltanet_steps, ssm_out. */
static int q35_linear_attention(ref_engine *e, layer_w *lw, int staged) {
    const int64_t D = e->dim, KD = e->lin_nk * e->lin_hk, VD = e->lin_nv * e->lin_hv, CD = 2 * KD + VD;
    ref_rmsnorm(e->xb, e->x, lw->attn_norm, D, e->rms_eps);
    if (matmul_mode(e, staged, e->hy_qkv, e->xb, &lw->in_qkv, D, CD) ||
        matmul_mode(e, staged, e->hy_z, e->xb, &lw->in_z, D, VD) ||
        matmul_mode(e, staged, e->hy_b, e->xb, &lw->in_b, D, e->lin_nv) ||
        matmul_mode(e, staged, e->hy_a, e->xb, &lw->in_a, D, e->lin_nv))
        return -1;
    if (ref_deltanet_steps((int)e->lin_nk, (int)e->lin_nv, (int)e->lin_hk, (int)e->lin_hv, (int)e->lin_kernel,
                           e->rms_eps, 1, e->hy_qkv, e->hy_z, e->hy_b, e->hy_a, lw->conv_w, lw->ssm_a, lw->dt_bias,
                           lw->ssm_norm, lw->conv_state, lw->rec_state, e->hy_out))
        return -1;
    if (matmul_mode(e, staged, e->xb2, e->hy_out, &lw->ssm_out, VD, D)) return -1;
    for (int64_t i = 0; i < D; i++) e->x[i] += e->xb2[i];
    return 0;
}

static const float *forward_impl(ref_engine *e, int token, int pos, int staged, int logits) {
    if (pos < 0 || pos >= e->seq_len) {
        snprintf(g_err, sizeof g_err, "forward: pos=%d out of range (seq_len=%lld)", pos, (long long)e->seq_len);
        return NULL;
    }
    if (token < 0 || token >= e->vocab_size) {
        snprintf(g_err, sizeof g_err, "forward: token=%d out of range (vocab=%lld)", token, (long long)e->vocab_size);
        return NULL;
    }
    int64_t dim = e->dim, hidden_dim = e->hidden_dim, head_dim = e->head_dim, n_heads = e->n_heads;
    int64_t n_kv_heads = e->n_kv_heads, seq_len = e->seq_len, kv_dim = n_kv_heads * head_dim;
    int64_t kv_mul = n_heads / n_kv_heads, att_head_dim = n_heads * head_dim;
    float eps = e->rms_eps;
    mm_pool *P = e->pool;

    /* get_embedding_row, infer/forward.odin:12-15 */
    int64_t rb = ref_row_byte_size(e->token_embedding.kind, dim);
    ref_dequant_row(e->token_embedding.kind, e->token_embedding.data + (int64_t)token * rb, dim, e->x);

    for (int64_t l = 0; l < e->n_layers; l++) {
        layer_w *lw = &e->layers[l];
        if (lw->kind == 1 && q35_full_attention(e, lw, pos, staged)) return NULL;
        if (lw->kind == 2 && q35_linear_attention(e, lw, staged)) return NULL;
        if (lw->kind != 0) goto ffn;
        {
        int64_t loff = l * seq_len * kv_dim;
        float *k_slice = e->key_cache + loff + (int64_t)pos * kv_dim;
        float *v_slice = e->value_cache + loff + (int64_t)pos * kv_dim;
        /* in f16 mode K/V are formed in f32 temporaries and rounded on store */
        float *kk = e->kv_f16 ? e->ktmp : k_slice;
        float *vv = e->kv_f16 ? e->vtmp : v_slice;

        ref_rmsnorm(e->xb, e->x, lw->attn_norm, dim, eps);
#define MM(out, in, t, n, d)                                                      \
    do {                                                                          \
        if (!staged) matmul_t(P, out, in, (t).kind, (t).data, n, d);              \
        else if (matmul_staged(e, out, in, (t).kind, (t).data, n, d)) return NULL; \
    } while (0)
        MM(e->q, e->xb, lw->wq, dim, att_head_dim);
        MM(kk, e->xb, lw->wk, dim, kv_dim);
        MM(vv, e->xb, lw->wv, dim, kv_dim);

        /* RoPE + per-head Q/K RMSNorm, infer/forward.odin:57-85 */
        for (int64_t h = 0; h < n_heads; h++) {
            float *q = e->q + h * head_dim;
            ref_rmsnorm(q, q, lw->q_norm, head_dim, eps);
            if (h < n_kv_heads) {
                float *k = kk + h * head_dim;
                ref_rmsnorm(k, k, lw->k_norm, head_dim, eps);
            }
            for (int64_t i = 0; i < head_dim / 2; i++) {
                float freq = 1.0f / powf(e->rope_freq, (float)i / (float)(head_dim / 2));
                float fcr = cosf((float)pos * freq);
                float fci = sinf((float)pos * freq);
                float x_q = q[i], y_q = q[i + head_dim / 2];
                q[i] = x_q * fcr - y_q * fci;
                q[i + head_dim / 2] = x_q * fci + y_q * fcr;
                if (h < n_kv_heads) {
                    float *k = kk + h * head_dim;
                    float x_k = k[i], y_k = k[i + head_dim / 2];
                    k[i] = x_k * fcr - y_k * fci;
                    k[i + head_dim / 2] = x_k * fci + y_k * fcr;
                }
            }
        }
        if (e->kv_f16) {
            for (int64_t i = 0; i < kv_dim; i++) {
                k_slice[i] = ref_f16_to_f32(ref_f32_to_f16(kk[i]));
                v_slice[i] = ref_f16_to_f32(ref_f32_to_f16(vv[i]));
            }
        }

        /* multihead attention, infer/forward.odin:87-115 */
        for (int64_t h = 0; h < n_heads; h++) {
            float *q = e->q + h * head_dim;
            float *att = e->att + h * seq_len;
            for (int64_t t = 0; t <= pos; t++) {
                const float *k = e->key_cache + loff + t * kv_dim + (h / kv_mul) * head_dim;
                float score = 0.0f;
                for (int64_t i = 0; i < head_dim; i++) score += q[i] * k[i];
                att[t] = score / sqrtf((float)head_dim);
            }
            ref_softmax(att, (int64_t)pos + 1);
            float *xb3 = e->xb3 + h * head_dim;
            for (int64_t i = 0; i < head_dim; i++) xb3[i] = 0.0f;
            for (int64_t t = 0; t <= pos; t++) {
                const float *v = e->value_cache + loff + t * kv_dim + (h / kv_mul) * head_dim;
                float a = att[t];
                for (int64_t i = 0; i < head_dim; i++) xb3[i] += a * v[i];
            }
        }

        MM(e->xb2, e->xb3, lw->wo, att_head_dim, dim);
        for (int64_t i = 0; i < dim; i++) e->x[i] += e->xb2[i];
        }
    ffn:
        ref_rmsnorm(e->xb, e->x, lw->ffn_norm, dim, eps);
        if (lw->moe) { /* routed experts (+ shared expert) */
            e->cur_pos = pos;
            e->cur_layer = l;
            moe_ffn_layer(e, lw, e->xb, e->mo_y);
            for (int64_t i = 0; i < dim; i++) e->x[i] += e->mo_y[i];
            continue;
        }
        if (e->arch == 2) { /* mlp_layer, qwen3_5/forward.odin:227-243 */
            if (matmul_mode(e, staged, e->hb, e->xb, &lw->w1, dim, hidden_dim) ||
                matmul_mode(e, staged, e->hb2, e->xb, &lw->w3, dim, hidden_dim))
                return NULL;
            for (int64_t i = 0; i < hidden_dim; i++) e->hb2[i] = ref_silu(e->hb[i]) * e->hb2[i];
            if (matmul_mode(e, staged, e->xb, e->hb2, &lw->w2, hidden_dim, dim)) return NULL;
            for (int64_t i = 0; i < dim; i++) e->x[i] += e->xb[i];
            continue;
        }
        MM(e->hb, e->xb, lw->w1, dim, hidden_dim);
        MM(e->hb2, e->xb, lw->w3, dim, hidden_dim);
        for (int64_t i = 0; i < hidden_dim; i++) { /* infer/forward.odin:128-132 */
            float val = e->hb[i];
            val *= 1.0f / (1.0f + expf(-val));
            val *= e->hb2[i];
            e->hb2[i] = val;
        }
        MM(e->xb, e->hb2, lw->w2, hidden_dim, dim);
#undef MM
        for (int64_t i = 0; i < dim; i++) e->x[i] += e->xb[i];
    }

    if (!logits) return e->logits;
    ref_rmsnorm(e->x, e->x, e->output_norm, dim, eps);
    matmul_t(P, e->logits, e->x, e->output.kind, e->output.data, dim, e->vocab_size);
    return e->logits;
}

/* forward (infer/forward.odin:17-146).  Returns the engine-owned logits, or
 * NULL (with ref_last_error) where the reference prints and exits. */
EXPORT const float *ref_engine_forward(void *h, int token, int pos) {
    return forward_impl((ref_engine *)h, token, pos, 0, 1);
}

/* engine_forward_batch (qwen3_5/engine.odin:61-93): chunks of up to
 * MAX_BATCH_T = 512 tokens (qwen3_5/metal.odin:22), cut to a multiple of 8, through
 * the batched path (staged projections, logits of the chunk's last token);
 * the trailing 1-7 tokens one at a time through forward.  In the batched path
 * of every layout the attention / DeltaNet projections and a dense MLP are
 * staged (forward_gpu_batch, qwen3_5/metal.odin:1510-1634); the routed-expert FFN,
 * which the reference does not have, stays in f32 (router, experts and
 * shared expert as the per-token path).  Returns the last token's logits, or
 * NULL. */
EXPORT const float *ref_engine_prefill(void *h, const int *tokens, int n, int pos0) {
    ref_engine *e = (ref_engine *)h;
    if (n <= 0) {
        snprintf(g_err, sizeof g_err, "prefill: no tokens");
        return NULL;
    }
    const float *out = NULL;
    int i = 0;
    while (i < n) {
        int rem = n - i;
        if (rem >= 8) {
            int chunk = rem < 512 ? rem : 512;
            chunk -= chunk % 8;
            for (int t = 0; t < chunk; t++)
                if (!(out = forward_impl(e, tokens[i + t], pos0 + i + t, 1, t == chunk - 1))) return NULL;
            i += chunk;
        } else {
            if (!(out = forward_impl(e, tokens[i], pos0 + i, 0, 1))) return NULL;
            i += 1;
        }
    }
    return out;
}

/* engine_verify_batch (qwen3_5/engine.odin:166-174): the tokens go through
 * the path of ref_engine_prefill (batched chunks of a multiple of 8 up to 512
 * with staged projections, the trailing 1-7 per token), and every position's
 * logits are kept: each token's final RMSNorm and classifier in f32
 * (metal_verify_batch_logits, qwen3_5/metal.odin:1707-1747: one enc_rmsnorm +
 * enc_gemv per row of the batch).  Returns [n][vocab] (engine-owned, valid
 * until the next call), or NULL. */
EXPORT const float *ref_engine_verify_batch(void *h, const int *tokens, int n, int pos0) {
    ref_engine *e = (ref_engine *)h;
    if (n <= 0) {
        snprintf(g_err, sizeof g_err, "verify_batch: no tokens");
        return NULL;
    }
    if (n > e->vf_rows) {
        float *b = (float *)realloc(e->vf, (size_t)n * (size_t)e->vocab_size * sizeof(float));
        if (!b) {
            snprintf(g_err, sizeof g_err, "verify_batch: out of memory");
            return NULL;
        }
        e->vf = b;
        e->vf_rows = n;
    }
    int i = 0;
    while (i < n) {
        int rem = n - i, chunk = 1, staged = 0;
        if (rem >= 8) {
            chunk = rem < 512 ? rem : 512;
            chunk -= chunk % 8;
            staged = 1;
        }
        for (int t = 0; t < chunk; t++) {
            const float *out = forward_impl(e, tokens[i + t], pos0 + i + t, staged, 1);
            if (!out) return NULL;
            memcpy(e->vf + (size_t)(i + t) * (size_t)e->vocab_size, out, (size_t)e->vocab_size * sizeof(float));
        }
        i += chunk;
    }
    return e->vf;
}

/* Test hook: start (on != 0; all margins NAN) or stop recording the routing
 * boundary margins; ref_engine_route_margins returns the [seq_len][n_layers]
 * table (NULL when not recording). */
EXPORT int ref_engine_route_log(void *h, int on) {
    ref_engine *e = (ref_engine *)h;
    free(e->rt_margin);
    e->rt_margin = NULL;
    if (!on) return 0;
    const size_t n = (size_t)e->seq_len * (size_t)e->n_layers;
    e->rt_margin = (float *)malloc(n * sizeof(float));
    if (!e->rt_margin) return -1;
    for (size_t i = 0; i < n; i++) e->rt_margin[i] = NAN;
    return 0;
}
EXPORT const float *ref_engine_route_margins(void *h) { return ((ref_engine *)h)->rt_margin; }

/* Hidden state after the final norm (test hook for layer-level checks). */
EXPORT const float *ref_engine_hidden(void *h) { return ((ref_engine *)h)->x; }

/* ---------------------------------------------------------------- sampler --
 * sampler/sampler.odin:68-199 without the grammar mask.  slice.sort_by
 * (:118) leaves equal probabilities in an unspecified order; here they keep
 * index order (the comparator breaks ties by index). */

static uint32_t ref_random_u32(uint64_t *state) { /* :68-73 */
    *state ^= *state >> 12;
    *state ^= *state << 25;
    *state ^= *state >> 27;
    return (uint32_t)((*state * 0x2545F4914F6CDD1Dull) >> 32);
}

EXPORT float ref_random_f32(uint64_t *state) { return (float)(ref_random_u32(state) >> 8) / 16777216.0f; }

static int64_t ref_sample_mult(const float *p, int64_t n, float coin) { /* :91-100 */
    float cdf = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        cdf += p[i];
        if (coin < cdf) return i;
    }
    return n - 1;
}

typedef struct { float prob; int64_t index; } prob_index;

static int prob_index_cmp(const void *a, const void *b) {
    const prob_index *x = (const prob_index *)a, *y = (const prob_index *)b;
    if (x->prob > y->prob) return -1;
    if (x->prob < y->prob) return 1;
    return x->index < y->index ? -1 : x->index > y->index;
}

static int64_t ref_sample_topp(const float *p, int64_t n, float topp, prob_index *pi, float coin) { /* :106-139 */
    int64_t n0 = 0;
    float cutoff = (1.0f - topp) / (float)(n - 1);
    for (int64_t i = 0; i < n; i++)
        if (p[i] >= cutoff) {
            pi[n0].index = i;
            pi[n0].prob = p[i];
            n0++;
        }
    qsort(pi, (size_t)n0, sizeof *pi, prob_index_cmp);
    float cumulative_prob = 0.0f;
    int64_t last_idx = n0 - 1;
    for (int64_t i = 0; i < n0; i++) {
        cumulative_prob += pi[i].prob;
        if (cumulative_prob > topp) {
            last_idx = i;
            break;
        }
    }
    float r = coin * cumulative_prob;
    float cdf = 0.0f;
    for (int64_t i = 0; i <= last_idx; i++) {
        cdf += pi[i].prob;
        if (r < cdf) return pi[i].index;
    }
    return pi[last_idx].index;
}

/* sample (:141-199): logits are modified in place, as the reference's are. */
EXPORT int64_t ref_sample(float *logits, int64_t n, float temperature, float topp, float penalty,
                          const int32_t *last, int n_last, uint64_t *rng) {
    if (penalty != 1.0f && n_last > 0) {
        int32_t seen[64];
        int ns = 0;
        for (int i = 0; i < n_last; i++) {
            int32_t tok = last[i];
            if (tok < 0 || tok >= n) continue;
            int dup = 0;
            for (int j = 0; j < ns; j++) dup |= seen[j] == tok;
            if (dup) continue;
            if (ns < 64) seen[ns++] = tok;
            if (logits[tok] > 0) logits[tok] /= penalty;
            else logits[tok] *= penalty;
        }
    }
    if (temperature == 0.0f) return ref_argmax(logits, n);
    for (int64_t i = 0; i < n; i++) logits[i] /= temperature;
    ref_softmax(logits, n);
    float coin = ref_random_f32(rng);
    if (topp <= 0 || topp >= 1) return ref_sample_mult(logits, n, coin);
    prob_index *pi = (prob_index *)malloc((size_t)n * sizeof *pi);
    if (!pi) return -1;
    int64_t r = ref_sample_topp(logits, n, topp, pi, coin);
    free(pi);
    return r;
}

/* record_token (:50-56) with its default window 64; last has room for 65 */
EXPORT void ref_record_token(int32_t *last, int *n_last, int32_t token, float penalty) {
    if (penalty == 1.0f) return;
    last[(*n_last)++] = token;
    while (*n_last > 64) {
        memmove(last, last + 1, (size_t)(*n_last - 1) * sizeof *last);
        (*n_last)--;
    }
}

/* ------------------------------------------------------ state persistence --
 * engine_reset_state (qwen3_5/engine.odin:112-132) and the .oikv v1 file of
 * qwen3_5/kv_persist.odin:1-381: cpu_save_kv (:218-265) / cpu_load_kv
 * (:267-336) for the f32 caches of the dense layers, metal_save_kv /
 * metal_load_kv's head-major f16 conversion (qwen3_5/metal.odin:780-962) for
 * the f16 caches of the Qwen3.5 full-attention layers.  The header is the 60
 * bytes write_header emits (kv_persist.odin:141-156); the checksum is CRC-32
 * (IEEE, reflected 0xEDB88320) over header + body, appended last. */

EXPORT void ref_engine_reset_state(void *h) {
    ref_engine *e = (ref_engine *)h;
    int64_t kv_dim = e->n_kv_heads * e->head_dim, conv_dim = 2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv;
    memset(e->key_cache, 0, (size_t)(e->n_layers * e->seq_len * kv_dim) * 4);
    memset(e->value_cache, 0, (size_t)(e->n_layers * e->seq_len * kv_dim) * 4);
    for (int64_t l = 0; l < e->n_layers; l++) {
        layer_w *lw = &e->layers[l];
        if (lw->kind == 2) {
            memset(lw->conv_state, 0, (size_t)(conv_dim * (e->lin_kernel - 1)) * 4);
            memset(lw->rec_state, 0, (size_t)(e->lin_nv * e->lin_hk * e->lin_hv) * 4);
        } else if (lw->kind == 1) {
            memset(lw->kc16, 0, (size_t)(e->n_kv_heads * e->seq_len * e->head_dim) * 2);
            memset(lw->vc16, 0, (size_t)(e->n_kv_heads * e->seq_len * e->head_dim) * 2);
        }
    }
}

static uint32_t kv_crc_update(uint32_t crc, const uint8_t *p, size_t n) {
    /* bitwise form of the reflected CRC-32 (crc holds the complemented register) */
    for (size_t i = 0; i < n; i++) {
        crc ^= p[i];
        for (int k = 0; k < 8; k++) crc = (crc >> 1) ^ (0xEDB88320u & (0u - (crc & 1u)));
    }
    return crc;
}

/* model_fingerprint, kv_persist.odin:74-93 */
static uint64_t kv_fingerprint(const ref_engine *e) {
    uint64_t h = 0xcbf29ce484222325ull;
    int64_t f[11] = {e->dim, e->n_layers, e->n_heads, e->n_kv_heads, e->head_dim, e->lin_nk,
                     e->lin_nv, e->lin_hk, e->lin_hv, e->lin_kernel, e->vocab_size};
    for (int i = 0; i < 11; i++) h = (h ^ (uint64_t)f[i]) * 0x100000001b3ull;
    return h;
}

/* 2 = KV_ARCH_QWEN3_5 (kv_persist.odin:53); 1 and 3 for the layouts the reference does not persist */
static uint32_t kv_arch(const ref_engine *e) { return e->arch == 2 ? 2u : e->arch == 1 ? 3u : 1u; }

typedef struct { FILE *f; uint32_t crc; int bad; } kv_out;

static void kv_put(kv_out *o, const void *p, size_t n) {
    o->crc = kv_crc_update(o->crc, (const uint8_t *)p, n);
    if (fwrite(p, 1, n, o->f) != n) o->bad = 1;
}
static void kv_put_u32(kv_out *o, uint32_t v) {
    uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    kv_put(o, b, 4);
}

static void kv_header_fields(const ref_engine *e, uint32_t n_valid, uint32_t out[10], int64_t *n_full, int64_t *n_lin) {
    *n_full = *n_lin = 0;
    for (int64_t l = 0; l < e->n_layers; l++) {
        if (e->layers[l].kind == 2) (*n_lin)++;
        else (*n_full)++;
    }
    uint32_t v[10] = {n_valid, (uint32_t)e->seq_len, (uint32_t)*n_full, (uint32_t)*n_lin,
                      (uint32_t)(e->n_kv_heads * e->head_dim), (uint32_t)(2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv),
                      (uint32_t)e->lin_kernel, (uint32_t)e->lin_nv, (uint32_t)e->lin_hk, (uint32_t)e->lin_hv};
    memcpy(out, v, sizeof v);
}

/* K or V of attention layer l at positions [0, n) as f32 rows [n][kv_dim] */
static void kv_layer_rows(const ref_engine *e, int64_t l, int which, int64_t n, float *rows) {
    const layer_w *lw = &e->layers[l];
    int64_t kv_dim = e->n_kv_heads * e->head_dim, hd = e->head_dim;
    if (lw->kind == 0) { /* cpu_save_kv: the layer's [seq_len][kv_dim] slice */
        const float *src = (which ? e->value_cache : e->key_cache) + l * e->seq_len * kv_dim;
        memcpy(rows, src, (size_t)(n * kv_dim) * 4);
        return;
    }
    const uint16_t *c = which ? lw->vc16 : lw->kc16; /* metal_save_kv's conversion */
    for (int64_t kh = 0; kh < e->n_kv_heads; kh++)
        for (int64_t p = 0; p < n; p++)
            for (int64_t d = 0; d < hd; d++)
                rows[p * kv_dim + kh * hd + d] = ref_f16_to_f32(c[(kh * e->seq_len + p) * hd + d]);
}

EXPORT int ref_engine_save_kv(void *h, const char *path, int n_valid_pos) {
    ref_engine *e = (ref_engine *)h;
    if (n_valid_pos < 0 || n_valid_pos > e->seq_len) {
        snprintf(g_err, sizeof g_err, "kv: n_valid_pos %d > seq_len %lld", n_valid_pos, (long long)e->seq_len);
        return -1;
    }
    kv_out o = {fopen(path, "wb"), 0xFFFFFFFFu, 0};
    if (!o.f) { snprintf(g_err, sizeof g_err, "kv: cannot open %s for write", path); return -1; }
    uint32_t f[10];
    int64_t n_full, n_lin;
    kv_header_fields(e, (uint32_t)n_valid_pos, f, &n_full, &n_lin);
    kv_put_u32(&o, 0x4F494B56u);
    kv_put_u32(&o, 1);
    kv_put_u32(&o, kv_arch(e));
    uint64_t fp = kv_fingerprint(e);
    kv_put_u32(&o, (uint32_t)fp);
    kv_put_u32(&o, (uint32_t)(fp >> 32));
    for (int i = 0; i < 10; i++) kv_put_u32(&o, f[i]);
    int64_t kv_dim = e->n_kv_heads * e->head_dim;
    float *rows = (float *)malloc((size_t)(n_valid_pos * kv_dim + 1) * 4);
    for (int64_t l = 0; l < e->n_layers && rows; l++) {
        if (e->layers[l].kind == 2) continue;
        for (int which = 0; which < 2; which++) {
            kv_layer_rows(e, l, which, n_valid_pos, rows);
            kv_put(&o, rows, (size_t)(n_valid_pos * kv_dim) * 4);
        }
    }
    free(rows);
    int64_t conv_n = (2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv) * (e->lin_kernel > 0 ? e->lin_kernel - 1 : 0);
    int64_t rec_n = e->lin_nv * e->lin_hk * e->lin_hv;
    for (int64_t l = 0; l < e->n_layers; l++)
        if (e->layers[l].kind == 2) kv_put(&o, e->layers[l].conv_state, (size_t)conv_n * 4);
    for (int64_t l = 0; l < e->n_layers; l++)
        if (e->layers[l].kind == 2) kv_put(&o, e->layers[l].rec_state, (size_t)rec_n * 4);
    uint32_t crc = o.crc ^ 0xFFFFFFFFu;
    kv_put_u32(&o, crc);
    if (fclose(o.f) != 0) o.bad = 1;
    if (o.bad) { snprintf(g_err, sizeof g_err, "kv: write failed"); return -1; }
    return 0;
}

static int kv_fail(FILE *f, const char *msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    if (f) fclose(f);
    return -1;
}

/* Returns the restored n_valid_pos, or -1 (message in ref_last_error). */
EXPORT int ref_engine_load_kv(void *h, const char *path) {
    ref_engine *e = (ref_engine *)h;
    FILE *f = fopen(path, "rb");
    if (!f) return kv_fail(NULL, "kv: cannot open file");
    uint8_t hb[60];
    if (fread(hb, 1, 60, f) != 60) return kv_fail(f, "kv: header truncated");
    uint32_t w[15];
    for (int i = 0; i < 15; i++)
        w[i] = (uint32_t)hb[4 * i] | (uint32_t)hb[4 * i + 1] << 8 | (uint32_t)hb[4 * i + 2] << 16 |
               (uint32_t)hb[4 * i + 3] << 24;
    uint64_t fp = (uint64_t)w[3] | (uint64_t)w[4] << 32;
    uint32_t mine[10];
    int64_t n_full, n_lin;
    kv_header_fields(e, 0, mine, &n_full, &n_lin);
    if (w[0] != 0x4F494B56u) return kv_fail(f, "kv: bad magic");
    if (w[1] != 1) return kv_fail(f, "kv: version mismatch");
    if (w[2] != kv_arch(e)) return kv_fail(f, "kv: arch mismatch");
    if (fp != kv_fingerprint(e)) return kv_fail(f, "kv: fingerprint mismatch");
    if (w[6] != mine[1]) return kv_fail(f, "kv: seq_len mismatch");
    if (w[5] > mine[1]) return kv_fail(f, "kv: file n_valid_pos > engine seq_len");
    for (int i = 2; i < 10; i++)
        if (w[5 + i] != mine[i]) return kv_fail(f, "kv: layer dimensions differ");
    /* verify_crc32 over everything but the last 4 bytes, before touching the state */
    fseek(f, 0, SEEK_END);
    long size = ftell(f);
    if (size < 64) return kv_fail(f, "kv: file too short");
    rewind(f);
    uint32_t crc = 0xFFFFFFFFu;
    uint8_t buf[65536];
    long left = size - 4;
    while (left > 0) {
        size_t n = left > (long)sizeof buf ? sizeof buf : (size_t)left;
        if (fread(buf, 1, n, f) != n) return kv_fail(f, "kv: read failed");
        crc = kv_crc_update(crc, buf, n);
        left -= (long)n;
    }
    if (fread(buf, 1, 4, f) != 4) return kv_fail(f, "kv: read failed");
    uint32_t stored = (uint32_t)buf[0] | (uint32_t)buf[1] << 8 | (uint32_t)buf[2] << 16 | (uint32_t)buf[3] << 24;
    if ((crc ^ 0xFFFFFFFFu) != stored) return kv_fail(f, "kv: CRC mismatch — file corrupted");
    fseek(f, 60, SEEK_SET);
    int64_t n = w[5], kv_dim = e->n_kv_heads * e->head_dim, hd = e->head_dim;
    int64_t conv_dim = 2 * e->lin_nk * e->lin_hk + e->lin_nv * e->lin_hv;
    int64_t conv_n = conv_dim * (e->lin_kernel > 0 ? e->lin_kernel - 1 : 0), rec_n = e->lin_nv * e->lin_hk * e->lin_hv;
    if ((uint64_t)size != 60u + 8u * (uint64_t)(n_full * n * kv_dim) + 4u * (uint64_t)(n_lin * (conv_n + rec_n)) + 4u)
        return kv_fail(f, "kv: file size does not match its header");
    /* zero the caches, then read (cpu_load_kv :313-333; f16 caches round as metal_load_kv) */
    memset(e->key_cache, 0, (size_t)(e->n_layers * e->seq_len * kv_dim) * 4);
    memset(e->value_cache, 0, (size_t)(e->n_layers * e->seq_len * kv_dim) * 4);
    float *rows = (float *)malloc((size_t)(n * kv_dim + 1) * 4);
    if (!rows) return kv_fail(f, "kv: out of memory");
    for (int64_t l = 0; l < e->n_layers; l++) {
        layer_w *lw = &e->layers[l];
        if (lw->kind == 2) continue;
        for (int which = 0; which < 2; which++) {
            if (fread(rows, 4, (size_t)(n * kv_dim), f) != (size_t)(n * kv_dim)) { free(rows); return kv_fail(f, "kv: read failed"); }
            if (lw->kind == 0) {
                float *dst = (which ? e->value_cache : e->key_cache) + l * e->seq_len * kv_dim;
                for (int64_t i = 0; i < n * kv_dim; i++)
                    dst[i] = e->kv_f16 ? ref_f16_to_f32(ref_f32_to_f16(rows[i])) : rows[i];
            } else {
                uint16_t *c = which ? lw->vc16 : lw->kc16;
                memset(c, 0, (size_t)(e->n_kv_heads * e->seq_len * hd) * 2);
                for (int64_t kh = 0; kh < e->n_kv_heads; kh++)
                    for (int64_t p = 0; p < n; p++)
                        for (int64_t d = 0; d < hd; d++)
                            c[(kh * e->seq_len + p) * hd + d] = ref_f32_to_f16(rows[p * kv_dim + kh * hd + d]);
            }
        }
    }
    free(rows);
    for (int64_t l = 0; l < e->n_layers; l++)
        if (e->layers[l].kind == 2 && fread(e->layers[l].conv_state, 4, (size_t)conv_n, f) != (size_t)conv_n)
            return kv_fail(f, "kv: conv_states read failed");
    for (int64_t l = 0; l < e->n_layers; l++)
        if (e->layers[l].kind == 2 && fread(e->layers[l].rec_state, 4, (size_t)rec_n, f) != (size_t)rec_n)
            return kv_fail(f, "kv: recurrent_states read failed");
    fclose(f);
    return (int)n;
}

/* Batched prefill projection as the reference's MMQ kernels compute it
 * (gemm_harness/gemm_test.odin:97-135 gemm_q4k_f32, :297-337 gemm_q6k_f32,
 * qwen3_5/metal.odin:493-609): each weight row is dequantized (ggml/quant.odin,
 * dequant_row), rounded to f16 (the kernels stage A in half), multiplied by f16
 * activations and summed; the sum is taken in float64 here, as the harness's
 * CPU reference does (gemm_test.odin:838-851), so the GPU's f32 accumulation
 * is compared against the exact product of the staged operands.
 * x: [n][k] f16 bits (token-major), c: [n][m] (token-major). */
EXPORT int ref_gemm_f16(int kind, const uint8_t *w, int64_t m, int64_t k, const uint16_t *x, int64_t n,
                        double *c) {
    const int64_t rb = ref_row_byte_size(kind, k);
    if (rb <= 0) {
        snprintf(g_err, sizeof g_err, "gemm: unsupported type %d or row length %lld", kind, (long long)k);
        return -1;
    }
    float *row = malloc((size_t)k * sizeof(float));
    double *xd = malloc((size_t)(n * k) * sizeof(double));
    if (!row || !xd) {
        free(row);
        free(xd);
        snprintf(g_err, sizeof g_err, "gemm: out of memory");
        return -1;
    }
    for (int64_t i = 0; i < n * k; i++) xd[i] = ref_f16_to_f32(x[i]);
    for (int64_t r = 0; r < m; r++) {
        ref_dequant_row(kind, w + r * rb, k, row);
        for (int64_t j = 0; j < k; j++) row[j] = ref_f16_to_f32(ref_f32_to_f16(row[j]));
        for (int64_t t = 0; t < n; t++) {
            const double *xt = xd + t * k;
            double s = 0.0;
            for (int64_t j = 0; j < k; j++) s += (double)row[j] * xt[j];
            c[t * m + r] = s;
        }
    }
    free(row);
    free(xd);
    return 0;
}

/* ---------------------------------------------- Qwen3.5 gated DeltaNet --- */

/* qwen3_5/ops.odin:7-14 */
static float ref_sigmoid(float x) {
    if (x >= 0.0f) {
        float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    float z = expf(x);
    return z / (1.0f + z);
}
static float ref_silu(float x) { return x * ref_sigmoid(x); }
/* qwen3_5/ops.odin:20-24 */
static float ref_softplus(float x) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return 0.0f;
    return (float)log((double)(1.0f + expf(x)));
}
/* qwen3_5/ops.odin:26-37: eps is a floor on the norm */
static void ref_l2norm(float *o, const float *x, int64_t n, float eps) {
    float ss = 0.0f;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    float nrm = sqrtf(ss);
    float inv = 1.0f / (nrm > eps ? nrm : eps);
    for (int64_t i = 0; i < n; i++) o[i] = x[i] * inv;
}
/* qwen3_5/ops.odin:97-117 */
static void ref_conv1d_step(float *out, const float *in, float *state, const float *w, int64_t conv_dim, int kernel) {
    int km1 = kernel - 1;
    for (int64_t c = 0; c < conv_dim; c++) {
        const float *wr = w + c * kernel;
        float *sb = state + c * km1;
        float acc = wr[km1] * in[c];
        for (int k = 0; k < km1; k++) acc += wr[k] * sb[k];
        out[c] = ref_silu(acc);
        for (int k = 0; k < km1 - 1; k++) sb[k] = sb[k + 1];
        if (km1 > 0) sb[km1 - 1] = in[c];
    }
}
/* qwen3_5/ops.odin:120-153 */
EXPORT void ref_delta_step(float *out, float *state, const float *q, const float *k, const float *v, float beta,
                           float decay, int hk, int hv) {
    for (int64_t i = 0; i < (int64_t)hk * hv; i++) state[i] *= decay;
    float *delta = malloc((size_t)hv * sizeof(float));
    for (int j = 0; j < hv; j++) {
        float s = 0.0f;
        for (int i = 0; i < hk; i++) s += state[(int64_t)i * hv + j] * k[i];
        delta[j] = (v[j] - s) * beta;
    }
    for (int i = 0; i < hk; i++) {
        float ki = k[i];
        for (int j = 0; j < hv; j++) state[(int64_t)i * hv + j] += ki * delta[j];
    }
    for (int j = 0; j < hv; j++) {
        float s = 0.0f;
        for (int i = 0; i < hk; i++) s += state[(int64_t)i * hv + j] * q[i];
        out[j] = s;
    }
    free(delta);
}
EXPORT void ref_conv1d(float *out, const float *in, float *state, const float *w, int64_t conv_dim, int kernel) {
    ref_conv1d_step(out, in, state, w, conv_dim, kernel);
}
EXPORT void ref_l2norm_into(float *o, const float *x, int64_t n, float eps) { ref_l2norm(o, x, n, eps); }

/* forward_linear_layer (qwen3_5/forward.odin:172-219) from the projections
 * to the gated RMSNorm, for n_tokens consecutive tokens (states carried). */
EXPORT int ref_deltanet_steps(int n_kh, int n_vh, int hk, int hv, int kernel, float eps, int n_tokens,
                              const float *qkv, const float *z, const float *b, const float *a, const float *conv_w,
                              const float *a_decay, const float *dt_bias, const float *norm_w, float *conv_state,
                              float *rec_state, float *out) {
    if (n_kh <= 0 || n_vh <= 0 || hk <= 0 || hv <= 0 || kernel < 1 || n_tokens <= 0) {
        snprintf(g_err, sizeof g_err, "deltanet: bad dims");
        return -1;
    }
    int64_t key_dim = (int64_t)n_kh * hk, value_dim = (int64_t)n_vh * hv, conv_dim = 2 * key_dim + value_dim;
    float scale = 1.0f / sqrtf((float)hk);
    float *co = malloc((size_t)conv_dim * sizeof(float));
    float *ql = malloc((size_t)key_dim * sizeof(float));
    float *kl = malloc((size_t)key_dim * sizeof(float));
    for (int t = 0; t < n_tokens; t++) {
        const float *in = qkv + (int64_t)t * conv_dim;
        float *o = out + (int64_t)t * value_dim;
        ref_conv1d_step(co, in, conv_state, conv_w, conv_dim, kernel);
        for (int kh = 0; kh < n_kh; kh++) {
            ref_l2norm(ql + (int64_t)kh * hk, co + (int64_t)kh * hk, hk, 1e-6f);
            ref_l2norm(kl + (int64_t)kh * hk, co + key_dim + (int64_t)kh * hk, hk, 1e-6f);
            for (int i = 0; i < hk; i++) ql[(int64_t)kh * hk + i] *= scale;
        }
        for (int vh = 0; vh < n_vh; vh++) {
            int kh = vh % n_kh;
            float beta = ref_sigmoid(b[(int64_t)t * n_vh + vh]);
            float g = a_decay[vh] * ref_softplus(a[(int64_t)t * n_vh + vh] + dt_bias[vh]);
            float decay = expf(g);
            ref_delta_step(o + (int64_t)vh * hv, rec_state + (int64_t)vh * hk * hv, ql + (int64_t)kh * hk,
                           kl + (int64_t)kh * hk, co + 2 * key_dim + (int64_t)vh * hv, beta, decay, hk, hv);
        }
        for (int vh = 0; vh < n_vh; vh++) {
            float *oh = o + (int64_t)vh * hv;
            const float *zh = z + (int64_t)t * value_dim + (int64_t)vh * hv;
            ref_rmsnorm(oh, oh, norm_w, hv, eps);
            for (int i = 0; i < hv; i++) oh[i] *= ref_silu(zh[i]);
        }
    }
    free(co);
    free(ql);
    free(kl);
    return 0;
}

/* The chunked form of the delta rule for one value head and one chunk of C
 * tokens (qwen3_5/metal.odin:416-468 chunked_delta, the math of
 * delta_harness/delta_ref.odin:186-283): with cp[t] = g[0]..g[t] (the decays'
 * running product) and the chunk's state S at entry,
 *   d_t = beta_t v_t - beta_t cp[t] S^T k_t - sum_{i<t} beta_t (cp[t]/cp[i]) (k_t.k_i) d_i
 *   o_t = cp[t] S^T q_t + sum_{i<=t} (cp[t]/cp[i]) (q_t.k_i) d_i      (the i = t factor 1)
 *   S'  = cp[C-1] S + sum_i (cp[C-1]/cp[i]) k_i d_i^T
 * which equals C tokenwise steps (S *= g; d = (v - S^T k) beta; S += k d^T;
 * o = S^T q) up to rounding.  q, k [C][hk]; v, out [C][hv]; state [hk][hv]. */
EXPORT void ref_delta_chunk(float *out, float *state, const float *q, const float *k, const float *v,
                            const float *beta, const float *g, int C, int hk, int hv) {
    if (C <= 0 || hk <= 0 || hv <= 0) return;
    float *cp = malloc((size_t)C * sizeof(float));
    float *kkt = malloc((size_t)C * C * sizeof(float)), *kqt = malloc((size_t)C * C * sizeof(float));
    float *s0k = malloc((size_t)C * hv * sizeof(float)), *s0q = malloc((size_t)C * hv * sizeof(float));
    float *d = malloc((size_t)C * hv * sizeof(float));
    float acc = 1.0f;
    for (int t = 0; t < C; t++) {
        acc *= g[t];
        cp[t] = acc;
    }
    for (int t = 0; t < C; t++)
        for (int i = 0; i < C; i++) {
            float dk = 0.0f, dq = 0.0f;
            for (int a = 0; a < hk; a++) {
                dk += k[(int64_t)i * hk + a] * k[(int64_t)t * hk + a];
                dq += k[(int64_t)i * hk + a] * q[(int64_t)t * hk + a];
            }
            kkt[t * C + i] = dk;
            kqt[t * C + i] = dq;
        }
    for (int t = 0; t < C; t++)
        for (int j = 0; j < hv; j++) {
            float sk = 0.0f, sq = 0.0f;
            for (int a = 0; a < hk; a++) {
                sk += state[(int64_t)a * hv + j] * k[(int64_t)t * hk + a];
                sq += state[(int64_t)a * hv + j] * q[(int64_t)t * hk + a];
            }
            s0k[(int64_t)t * hv + j] = sk;
            s0q[(int64_t)t * hv + j] = sq;
        }
    for (int t = 0; t < C; t++)
        for (int j = 0; j < hv; j++)
            d[(int64_t)t * hv + j] = beta[t] * v[(int64_t)t * hv + j] - beta[t] * cp[t] * s0k[(int64_t)t * hv + j];
    for (int t = 0; t < C; t++)
        for (int i = 0; i < t; i++) {
            float L = beta[t] * (cp[t] / cp[i]) * kkt[t * C + i];
            for (int j = 0; j < hv; j++) d[(int64_t)t * hv + j] -= L * d[(int64_t)i * hv + j];
        }
    for (int t = 0; t < C; t++) {
        float *o = out + (int64_t)t * hv;
        for (int j = 0; j < hv; j++) o[j] = cp[t] * s0q[(int64_t)t * hv + j];
        for (int i = 0; i <= t; i++) {
            float w = (i < t ? cp[t] / cp[i] : 1.0f) * kqt[t * C + i];
            for (int j = 0; j < hv; j++) o[j] += w * d[(int64_t)i * hv + j];
        }
    }
    float cpC = cp[C - 1];
    for (int64_t x = 0; x < (int64_t)hk * hv; x++) state[x] *= cpC;
    for (int i = 0; i < C; i++) {
        float f = cp[C - 1] / cp[i];
        for (int a = 0; a < hk; a++) {
            float ka = f * k[(int64_t)i * hk + a];
            for (int j = 0; j < hv; j++) state[(int64_t)a * hv + j] += ka * d[(int64_t)i * hv + j];
        }
    }
    free(cp); free(kkt); free(kqt); free(s0k); free(s0q); free(d);
}

/* ref_deltanet_steps with the delta rule in chunks of `chunk` tokens (the last
 * chunk may be shorter): per token the conv, l2norm and gates as the tokenwise
 * form, per chunk and value head ref_delta_chunk, then per token the gated
 * RMSNorm. */
EXPORT int ref_deltanet_steps_chunked(int n_kh, int n_vh, int hk, int hv, int kernel, float eps, int n_tokens,
                                      int chunk, const float *qkv, const float *z, const float *b, const float *a,
                                      const float *conv_w, const float *a_decay, const float *dt_bias,
                                      const float *norm_w, float *conv_state, float *rec_state, float *out) {
    if (n_kh <= 0 || n_vh <= 0 || hk <= 0 || hv <= 0 || kernel < 1 || n_tokens <= 0 || chunk <= 0) {
        snprintf(g_err, sizeof g_err, "deltanet: bad dims");
        return -1;
    }
    int64_t key_dim = (int64_t)n_kh * hk, value_dim = (int64_t)n_vh * hv, conv_dim = 2 * key_dim + value_dim;
    float scale = 1.0f / sqrtf((float)hk);
    float *co = malloc((size_t)conv_dim * sizeof(float));
    float *ql = malloc((size_t)chunk * key_dim * sizeof(float)), *kl = malloc((size_t)chunk * key_dim * sizeof(float));
    float *vv = malloc((size_t)chunk * value_dim * sizeof(float));
    float *bt = malloc((size_t)chunk * n_vh * sizeof(float)), *gt = malloc((size_t)chunk * n_vh * sizeof(float));
    float *qh = malloc((size_t)chunk * hk * sizeof(float)), *kh_ = malloc((size_t)chunk * hk * sizeof(float));
    float *vh_ = malloc((size_t)chunk * hv * sizeof(float)), *oh = malloc((size_t)chunk * hv * sizeof(float));
    float *bh = malloc((size_t)chunk * sizeof(float)), *gh = malloc((size_t)chunk * sizeof(float));
    for (int t0 = 0; t0 < n_tokens; t0 += chunk) {
        int C = n_tokens - t0 < chunk ? n_tokens - t0 : chunk;
        for (int c = 0; c < C; c++) {
            int t = t0 + c;
            ref_conv1d_step(co, qkv + (int64_t)t * conv_dim, conv_state, conv_w, conv_dim, kernel);
            for (int kh = 0; kh < n_kh; kh++) {
                float *qd = ql + (int64_t)c * key_dim + (int64_t)kh * hk, *kd = kl + (int64_t)c * key_dim + (int64_t)kh * hk;
                ref_l2norm(qd, co + (int64_t)kh * hk, hk, 1e-6f);
                ref_l2norm(kd, co + key_dim + (int64_t)kh * hk, hk, 1e-6f);
                for (int i = 0; i < hk; i++) qd[i] *= scale;
            }
            memcpy(vv + (int64_t)c * value_dim, co + 2 * key_dim, (size_t)value_dim * sizeof(float));
            for (int vh = 0; vh < n_vh; vh++) {
                bt[c * n_vh + vh] = ref_sigmoid(b[(int64_t)t * n_vh + vh]);
                gt[c * n_vh + vh] = expf(a_decay[vh] * ref_softplus(a[(int64_t)t * n_vh + vh] + dt_bias[vh]));
            }
        }
        for (int vh = 0; vh < n_vh; vh++) {
            int kh = vh % n_kh;
            for (int c = 0; c < C; c++) {
                memcpy(qh + (int64_t)c * hk, ql + (int64_t)c * key_dim + (int64_t)kh * hk, (size_t)hk * sizeof(float));
                memcpy(kh_ + (int64_t)c * hk, kl + (int64_t)c * key_dim + (int64_t)kh * hk, (size_t)hk * sizeof(float));
                memcpy(vh_ + (int64_t)c * hv, vv + (int64_t)c * value_dim + (int64_t)vh * hv, (size_t)hv * sizeof(float));
                bh[c] = bt[c * n_vh + vh];
                gh[c] = gt[c * n_vh + vh];
            }
            ref_delta_chunk(oh, rec_state + (int64_t)vh * hk * hv, qh, kh_, vh_, bh, gh, C, hk, hv);
            for (int c = 0; c < C; c++)
                memcpy(out + (int64_t)(t0 + c) * value_dim + (int64_t)vh * hv, oh + (int64_t)c * hv,
                       (size_t)hv * sizeof(float));
        }
        for (int c = 0; c < C; c++)
            for (int vh = 0; vh < n_vh; vh++) {
                float *o = out + (int64_t)(t0 + c) * value_dim + (int64_t)vh * hv;
                const float *zh = z + (int64_t)(t0 + c) * value_dim + (int64_t)vh * hv;
                ref_rmsnorm(o, o, norm_w, hv, eps);
                for (int i = 0; i < hv; i++) o[i] *= ref_silu(zh[i]);
            }
    }
    free(co); free(ql); free(kl); free(vv); free(bt); free(gt);
    free(qh); free(kh_); free(vh_); free(oh); free(bh); free(gh);
    return 0;
}

/* ---------------------------------------- Qwen3.5 full-attention layer --- */

/* qwen3_5/ops.odin:163-168 */
EXPORT void ref_inv_freq(float theta, int rotary_dim, float *out) {
    float rd = (float)rotary_dim;
    for (int i = 0; i < rotary_dim / 2; i++) out[i] = 1.0f / powf(theta, (float)i / (rd / 2.0f));
}
/* qwen3_5/ops.odin:77-89: pairs (i, i + rotary_dim/2); dimensions past rotary_dim pass */
EXPORT void ref_mrope(float *v, int pos, const float *inv_freq, int rotary_dim) {
    int half = rotary_dim / 2;
    float pf = (float)pos;
    for (int i = 0; i < half; i++) {
        float angle = pf * inv_freq[i];
        float c = cosf(angle), s = sinf(angle);
        float x = v[i], y = v[i + half];
        v[i] = x * c - y * s;
        v[i + half] = x * s + y * c;
    }
}

/* The attention of forward_full_layer (qwen3_5/forward.odin:69-127) for
 * n_tokens tokens at pos0.. over an f16 cache (k/v rounded on store, as the
 * GPU path keeps them); caches are binary16 bits [n_kv][seq_len][head_dim]. */
EXPORT int ref_qwen35_attn_steps(int n_heads, int n_kv, int hd, int rotary_dim, int seq_len, float eps, int n_tokens,
                                 int pos0, const float *qproj, const float *k, const float *v, const float *q_norm,
                                 const float *k_norm, const float *inv_freq, uint16_t *kc, uint16_t *vc, float *out) {
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || hd <= 0 || rotary_dim < 0 || rotary_dim > hd ||
        n_tokens <= 0 || pos0 < 0 || pos0 + n_tokens > seq_len) {
        snprintf(g_err, sizeof g_err, "qwen35 attention: bad arguments");
        return -1;
    }
    int kv_mul = n_heads / n_kv;
    float att_scale = 1.0f / sqrtf((float)hd);
    float *q = malloc((size_t)n_heads * hd * sizeof(float));
    float *kk = malloc((size_t)n_kv * hd * sizeof(float));
    float *att = malloc((size_t)seq_len * sizeof(float));
    float *row = malloc((size_t)hd * sizeof(float));
    for (int t = 0; t < n_tokens; t++) {
        int pos = pos0 + t;
        const float *qp = qproj + (int64_t)t * n_heads * 2 * hd;
        for (int h = 0; h < n_heads; h++) ref_rmsnorm(q + (int64_t)h * hd, qp + (int64_t)h * 2 * hd, q_norm, hd, eps);
        for (int h = 0; h < n_kv; h++)
            ref_rmsnorm(kk + (int64_t)h * hd, k + ((int64_t)t * n_kv + h) * hd, k_norm, hd, eps);
        for (int h = 0; h < n_heads; h++) ref_mrope(q + (int64_t)h * hd, pos, inv_freq, rotary_dim);
        for (int h = 0; h < n_kv; h++) ref_mrope(kk + (int64_t)h * hd, pos, inv_freq, rotary_dim);
        for (int h = 0; h < n_kv; h++)
            for (int i = 0; i < hd; i++) {
                int64_t off = ((int64_t)h * seq_len + pos) * hd + i;
                kc[off] = ref_f32_to_f16(kk[(int64_t)h * hd + i]);
                vc[off] = ref_f32_to_f16(v[((int64_t)t * n_kv + h) * hd + i]);
            }
        for (int h = 0; h < n_heads; h++) {
            const float *qh = q + (int64_t)h * hd;
            int kh = h / kv_mul;
            for (int tt = 0; tt <= pos; tt++) {
                for (int i = 0; i < hd; i++) row[i] = ref_f16_to_f32(kc[((int64_t)kh * seq_len + tt) * hd + i]);
                att[tt] = ref_dot_f32(qh, row, hd) * att_scale;
            }
            ref_softmax(att, (int64_t)pos + 1);
            float *o = out + ((int64_t)t * n_heads + h) * hd;
            for (int i = 0; i < hd; i++) o[i] = 0.0f;
            for (int tt = 0; tt <= pos; tt++) {
                float a = att[tt];
                for (int i = 0; i < hd; i++) o[i] += a * ref_f16_to_f32(vc[((int64_t)kh * seq_len + tt) * hd + i]);
            }
            const float *gate = qp + (int64_t)h * 2 * hd + hd;
            for (int i = 0; i < hd; i++) o[i] *= ref_sigmoid(gate[i]);
        }
    }
    free(q); free(kk); free(att); free(row);
    return 0;
}

/* ------------------------------------------------- mixture of experts --- */

/* Routed-expert SwiGLU FFN for one token.  The reference has no MoE code; the
 * convention restated is HF Qwen3-MoE's: logits = router x (rows dequantized,
 * dot_f32 as matmul_t), p = softmax (qwen3_5/ops.odin:51-68 form), the top_k largest
 * (strict '>' scan: ties to the lower id, as sampler.odin:79-89), weights p or
 * p / sum, y = sum_k w_k down_e(silu(gate_e x) * up_e x), k in selection order. */
EXPORT int ref_moe_ffn(int E, int top_k, int dim, int inter, int norm, int rtype, const uint8_t *router, int etype,
                       const uint8_t *gate, const uint8_t *up, const uint8_t *down, const float *x, float *y,
                       int *ids, float *wout) {
    if (E <= 0 || top_k <= 0 || top_k > E || dim <= 0 || inter <= 0) {
        snprintf(g_err, sizeof g_err, "moe: bad dims");
        return -1;
    }
    int64_t rb = ref_row_byte_size(rtype, dim), gb = ref_row_byte_size(etype, dim), db = ref_row_byte_size(etype, inter);
    float *p = malloc((size_t)E * sizeof(float)), *row = malloc((size_t)(dim > inter ? dim : inter) * sizeof(float));
    float *h = malloc((size_t)top_k * inter * sizeof(float)), *w = malloc((size_t)top_k * sizeof(float));
    for (int e = 0; e < E; e++) {
        ref_dequant_row(rtype, router + e * rb, dim, row);
        p[e] = ref_dot_f32(row, x, dim);
    }
    ref_softmax(p, E);
    float sum = 0.0f;
    for (int k = 0; k < top_k; k++) {
        int best = -1;
        for (int e = 0; e < E; e++)
            if (p[e] >= 0.0f && (best < 0 || p[e] > p[best])) best = e;
        if (best < 0) { /* NaN probabilities rank nothing: expert 0 at weight 0, as the device does */
            ids[k] = 0;
            w[k] = 0.0f;
            continue;
        }
        ids[k] = best;
        w[k] = p[best];
        sum += p[best];
        p[best] = -1.0f;
    }
    for (int k = 0; k < top_k; k++) wout[k] = norm ? w[k] / sum : w[k];
    for (int k = 0; k < top_k; k++) {
        int64_t e = ids[k];
        for (int r = 0; r < inter; r++) {
            ref_dequant_row(etype, gate + (e * inter + r) * gb, dim, row);
            float g = ref_dot_f32(row, x, dim);
            ref_dequant_row(etype, up + (e * inter + r) * gb, dim, row);
            float u = ref_dot_f32(row, x, dim);
            h[(int64_t)k * inter + r] = ref_silu(g) * u;
        }
    }
    for (int r = 0; r < dim; r++) {
        float acc = 0.0f;
        for (int k = 0; k < top_k; k++) {
            int64_t e = ids[k];
            ref_dequant_row(etype, down + (e * dim + r) * db, inter, row);
            acc += wout[k] * ref_dot_f32(row, h + (int64_t)k * inter, inter);
        }
        y[r] = acc;
    }
    free(p); free(row); free(h); free(w);
    return 0;
}
