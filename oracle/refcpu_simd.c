/*
 * refcpu_simd.c — the reference's CPU kernels restated with x86 intrinsics and
 * its worker pool restated with pthreads. TEST/BENCH INFRASTRUCTURE ONLY: this
 * is the "restated reference CPU path" that bench.py times as cpu_baseline.
 * It is never part of the product library.
 *
 * Kernels (each mirrors one Go-assembler routine instruction for instruction
 * where the arithmetic is concerned):
 *   q8q8_row_vnni   vnni_amd64.s:41-84       VPDPBUSD(w^0x80, xq) - 128·Σxq
 *   q8q8_row_avx2   q8q8_row_amd64.s:16-58   VPMOVSXBW + VPMADDWD
 *   q4q8_row_avx2   q4q8_row_amd64.s:24-88   VPMADDUBSW, 4 rotating FMA accumulators
 *   q41q8_row_vnni  q41q8_vnni_amd64.s:17-74
 *   q41q8_row_avx2  q41q8_row_amd64.s:25-83
 * Drivers mirror q8q8.go:147-246, q4q8.go:49-101, q41q8.go:20-60,
 * kquant_kernels.go:159-174 and float32_ops.go:427-436 (Q5_0 stays scalar Go
 * in the reference, so it uses ref_q5_row). The pool mirrors parallel.go:
 * nWorkers = NumCPU (<=8), NumCPU-2 (<=18) else 16 (parallel.go:35-43);
 * chunk = ceil(n / (4*nWorkers)) claimed by an atomic cursor, the caller
 * participates (parallel.go:301-346, 249-267); idle workers spin, then park.
 * Kernel choice is what the reference picks on a VNNI host (vnni_amd64.go:12-21,
 * q41q8_vnni_amd64.go:15-20): VNNI for Q8_0 and Q4_1 when the CPU has AVX-VNNI,
 * else the fused AVX2 kernels; fused AVX2 for Q4_0.
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "refcpu.h"

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline int32_t hsum_epi32(__m256i v) {
    __m128i a = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    a = _mm_add_epi32(a, _mm_shuffle_epi32(a, 0x4e));
    a = _mm_add_epi32(a, _mm_shuffle_epi32(a, 0xb1));
    return _mm_cvtsi128_si32(a);
}

static inline float cvtph(uint16_t h) { return _mm_cvtss_f32(_mm_cvtph_ps(_mm_cvtsi32_si128(h))); }

/* ------------------------------------------------------------ kernels ---- */

__attribute__((target("avx2,avxvnni")))
static float q8q8_row_vnni(const uint8_t *w, const int8_t *xq, const float *cmb, const int32_t *corr, int groups) {
    const __m256i mask = _mm256_set1_epi8((char)0x80);
    float acc = 0.0f;
    for (int g = 0; g < groups; g++) {
        __m256i wv = _mm256_xor_si256(_mm256_loadu_si256((const __m256i *)(w + 2)), mask);
        __m256i xv = _mm256_loadu_si256((const __m256i *)xq);
        __m256i s = _mm256_dpbusd_avx_epi32(_mm256_setzero_si256(), wv, xv);
        int32_t isum = hsum_epi32(s) - corr[g];
        float t = (float)isum * cmb[g];
        acc = acc + t;
        w += 34; xq += 32;
    }
    return acc;
}

static float q8q8_row_avx2(const uint8_t *w, const int8_t *xq, const float *cmb, int groups) {
    float acc = 0.0f;
    for (int g = 0; g < groups; g++) {
        __m256i w0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + 2)));
        __m256i w1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + 18)));
        __m256i x0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)xq));
        __m256i x1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(xq + 16)));
        __m256i p = _mm256_add_epi32(_mm256_madd_epi16(w0, x0), _mm256_madd_epi16(w1, x1));
        float t = (float)hsum_epi32(p) * cmb[g];
        acc = acc + t;
        w += 34; xq += 32;
    }
    return acc;
}

static float q4q8_row_avx2(const uint8_t *w, const int8_t *xq, const float *xs, const int32_t *corr, int groups) {
    const __m256i ones = _mm256_set1_epi16(1);
    const __m128i lo = _mm_set1_epi8(0x0f);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
#define Q4BODY(A)                                                                         \
    do {                                                                                  \
        __m128i raw = _mm_loadu_si128((const __m128i *)(w + 2));                          \
        __m128i l = _mm_and_si128(raw, lo);                                               \
        __m128i h = _mm_and_si128(_mm_srli_epi16(raw, 4), lo);                            \
        __m256i nib = _mm256_inserti128_si256(_mm256_castsi128_si256(l), h, 1);           \
        __m256i x = _mm256_loadu_si256((const __m256i *)xq);                              \
        __m256i p = _mm256_madd_epi16(_mm256_maddubs_epi16(nib, x), ones);                \
        p = _mm256_sub_epi32(p, _mm256_castsi128_si256(_mm_cvtsi32_si128(*corr)));        \
        __m256 pf = _mm256_cvtepi32_ps(p);                                                \
        float dxs = cvtph(rd16(w)) * *xs;                                                 \
        acc[A] = _mm256_fmadd_ps(pf, _mm256_set1_ps(dxs), acc[A]);                        \
        w += 18; xq += 32; xs += 1; corr += 1;                                            \
    } while (0)
    int g = groups;
    while (g >= 4) { Q4BODY(0); Q4BODY(1); Q4BODY(2); Q4BODY(3); g -= 4; }
    while (g > 0) { Q4BODY(0); g--; }
#undef Q4BODY
    __m256 a = _mm256_add_ps(_mm256_add_ps(acc[0], acc[1]), _mm256_add_ps(acc[2], acc[3]));
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

#define Q41_TAIL(qsum)                                       \
    do {                                                     \
        float d = cvtph(rd16(w)), m = cvtph(rd16(w + 2));     \
        float t = (float)(qsum) * d;                         \
        float u = (float)(*sxq) * m;                         \
        t = t + u;                                           \
        t = t * *xs;                                         \
        acc = acc + t;                                       \
        w += 20; xq += 32; xs += 1; sxq += 1;                \
    } while (0)

__attribute__((target("avx2,avxvnni")))
static float q41q8_row_vnni(const uint8_t *w, const int8_t *xq, const float *xs, const int32_t *sxq, int groups) {
    const __m128i lo = _mm_set1_epi8(0x0f);
    float acc = 0.0f;
    for (int g = 0; g < groups; g++) {
        __m128i raw = _mm_loadu_si128((const __m128i *)(w + 4));
        __m256i nib = _mm256_inserti128_si256(_mm256_castsi128_si256(_mm_and_si128(raw, lo)),
                                              _mm_and_si128(_mm_srli_epi16(raw, 4), lo), 1);
        __m256i s = _mm256_dpbusd_avx_epi32(_mm256_setzero_si256(), nib,
                                            _mm256_loadu_si256((const __m256i *)xq));
        Q41_TAIL(hsum_epi32(s));
    }
    return acc;
}

static float q41q8_row_avx2(const uint8_t *w, const int8_t *xq, const float *xs, const int32_t *sxq, int groups) {
    const __m128i lo = _mm_set1_epi8(0x0f);
    const __m256i ones = _mm256_set1_epi16(1);
    float acc = 0.0f;
    for (int g = 0; g < groups; g++) {
        __m128i raw = _mm_loadu_si128((const __m128i *)(w + 4));
        __m256i nib = _mm256_inserti128_si256(_mm256_castsi128_si256(_mm_and_si128(raw, lo)),
                                              _mm_and_si128(_mm_srli_epi16(raw, 4), lo), 1);
        __m256i p = _mm256_madd_epi16(_mm256_maddubs_epi16(nib, _mm256_loadu_si256((const __m256i *)xq)), ones);
        Q41_TAIL(hsum_epi32(p));
    }
    return acc;
}

/* --------------------------------------------------------------- pool ---- */

typedef void (*chunk_fn)(void *ctx, int start, int end);

static struct {
    int n_workers;
    pthread_t threads[64];
    atomic_ulong gen;
    atomic_long next_chunk, remaining;
    long num_chunks;
    int n, chunk;
    chunk_fn fn;
    void *ctx;
    pthread_mutex_t mu;
    pthread_cond_t cv;
    int started;
} pool = {.mu = PTHREAD_MUTEX_INITIALIZER, .cv = PTHREAD_COND_INITIALIZER};

static int num_cpu(void) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) return CPU_COUNT(&set);
    return 1;
}

int bl_default_workers(void) {
    int n = num_cpu();
    if (n <= 8) return n;
    if (n <= 18) return n - 2;
    return 16;
}

static void run_chunks(void) {
    long nc = pool.num_chunks;
    for (;;) {
        long c = atomic_fetch_add(&pool.next_chunk, 1);
        if (c >= nc) return;
        int start = (int)c * pool.chunk;
        int end = start + pool.chunk;
        if (end > pool.n) end = pool.n;
        pool.fn(pool.ctx, start, end);
        atomic_fetch_sub(&pool.remaining, 1);
    }
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

static void *worker(void *arg) {
    (void)arg;
    unsigned long last = atomic_load(&pool.gen);
    for (;;) {
        double idle = now_s();
        while (atomic_load(&pool.gen) == last) {
            for (int i = 0; i < 2048 && atomic_load(&pool.gen) == last; i++) _mm_pause();
            if (now_s() - idle > 50e-6) {
                pthread_mutex_lock(&pool.mu);
                while (atomic_load(&pool.gen) == last) pthread_cond_wait(&pool.cv, &pool.mu);
                pthread_mutex_unlock(&pool.mu);
            }
        }
        last = atomic_load(&pool.gen);
        run_chunks();
    }
    return NULL;
}

void bl_set_workers(int n) {
    if (pool.started) return;
    if (n < 1) n = 1;
    if (n > 64) n = 64;
    pool.n_workers = n;
}

int bl_workers(void) {
    if (!pool.n_workers) pool.n_workers = bl_default_workers();
    return pool.n_workers;
}

static void parallel_for(int n, chunk_fn fn, void *ctx) {
    int nw = bl_workers();
    if (nw <= 1 || n <= 1) { fn(ctx, 0, n); return; }
    if (!pool.started) {
        pool.started = 1;
        for (int i = 1; i < nw; i++) pthread_create(&pool.threads[i], NULL, worker, NULL);
    }
    int chunk = (n + nw * 4 - 1) / (nw * 4);
    if (chunk < 1) chunk = 1;
    pool.fn = fn;
    pool.ctx = ctx;
    pool.n = n;
    pool.chunk = chunk;
    pool.num_chunks = (n + chunk - 1) / chunk;
    atomic_store(&pool.next_chunk, 0);
    atomic_store(&pool.remaining, pool.num_chunks);
    pthread_mutex_lock(&pool.mu);
    atomic_fetch_add(&pool.gen, 1);
    pthread_cond_broadcast(&pool.cv);
    pthread_mutex_unlock(&pool.mu);
    run_chunks();
    while (atomic_load(&pool.remaining) > 0) _mm_pause();
}

/* ------------------------------------------------------------ drivers ---- */

int bl_has_vnni(void) { return __builtin_cpu_supports("avxvnni"); }

typedef struct {
    const uint8_t *raw;
    int N, G, M, K;
    const int8_t *xq;
    const float *xs;
    const int32_t *aux; /* corr or Σxq per (row, group) */
    const float *x;
    float *dst;
    int vnni;
} job_t;

static void q8_chunk(void *p, int js, int je) {
    job_t *J = (job_t *)p;
    float ws[4096], cmb[4096];
    for (int j = js; j < je; j++) {
        const uint8_t *row = J->raw + (size_t)j * J->G * 34;
        for (int g = 0; g < J->G; g++) ws[g] = ref_f16_to_f32_lut(rd16(row + (size_t)g * 34));
        for (int xi = 0; xi < J->M; xi++) {
            const float *xs = J->xs + (size_t)xi * J->G;
            for (int g = 0; g < J->G; g++) cmb[g] = ws[g] * xs[g];
            const int8_t *xq = J->xq + (size_t)xi * J->K;
            J->dst[(size_t)xi * J->N + j] = J->vnni
                ? q8q8_row_vnni(row, xq, cmb, J->aux + (size_t)xi * J->G, J->G)
                : q8q8_row_avx2(row, xq, cmb, J->G);
        }
    }
}

static void q4_chunk(void *p, int s, int e) {
    job_t *J = (job_t *)p;
    for (int idx = s; idx < e; idx++) {
        int xi = idx / J->N, j = idx % J->N;
        J->dst[idx] = q4q8_row_avx2(J->raw + (size_t)j * J->G * 18, J->xq + (size_t)xi * J->K,
                                    J->xs + (size_t)xi * J->G, J->aux + (size_t)xi * J->G, J->G);
    }
}

static void q41_chunk(void *p, int s, int e) {
    job_t *J = (job_t *)p;
    for (int idx = s; idx < e; idx++) {
        int xi = idx / J->N, j = idx % J->N;
        const uint8_t *row = J->raw + (size_t)j * J->G * 20;
        const int8_t *xq = J->xq + (size_t)xi * J->K;
        const float *xs = J->xs + (size_t)xi * J->G;
        const int32_t *sx = J->aux + (size_t)xi * J->G;
        J->dst[idx] = J->vnni ? q41q8_row_vnni(row, xq, xs, sx, J->G) : q41q8_row_avx2(row, xq, xs, sx, J->G);
    }
}

static void q5_chunk(void *p, int s, int e) {
    job_t *J = (job_t *)p;
    for (int idx = s; idx < e; idx++) {
        int xi = idx / J->N, j = idx % J->N;
        J->dst[idx] = ref_q5_row(J->raw + (size_t)j * J->G * 22, J->x + (size_t)xi * J->K, J->G);
    }
}

static int q41_pass(const uint8_t *raw, int N, int G, const float *x, int M, float *dst) {
    int K = G * 32;
    int8_t *xq = malloc((size_t)M * K);
    float *xs = malloc((size_t)M * G * 4);
    int32_t *sx = malloc((size_t)M * G * 4);
    if (!xq || !xs || !sx) { free(xq); free(xs); free(sx); return -1; }
    for (int r = 0; r < M; r++) ref_quantize_act_q8(x + (size_t)r * K, G, xq + (size_t)r * K, xs + (size_t)r * G);
    for (size_t i = 0; i < (size_t)M * G; i++) {
        int32_t s = 0;
        for (int k = 0; k < 32; k++) s += xq[i * 32 + k];
        sx[i] = s;
    }
    job_t J = {raw, N, G, M, K, xq, xs, sx, x, dst, bl_has_vnni()};
    parallel_for(M * N, q41_chunk, &J);
    free(xq); free(xs); free(sx);
    return 0;
}

/* Threaded SIMD modelMatmulQuantIntoF32 (float32_ops.go:379-460). */
int bl_matmul(const char *qtype, const uint8_t *raw, int N, int K, const float *x, int M, float *dst) {
    if (K % 32) return -1;
    int G = K / 32;
    if (!strcmp(qtype, "q4_1")) return q41_pass(raw, N, G, x, M, dst);
    if (!strcmp(qtype, "q5k1")) {
        float *tmp = malloc((size_t)M * N * 4);
        if (!tmp) return -1;
        int rc = q41_pass(raw, N, G, x, M, dst);
        if (!rc) rc = q41_pass(raw + (size_t)N * G * 20, N, G, x, M, tmp);
        for (size_t i = 0; !rc && i < (size_t)M * N; i++) dst[i] += tmp[i];
        free(tmp);
        return rc;
    }
    if (!strcmp(qtype, "q5")) {
        job_t J = {raw, N, G, M, K, NULL, NULL, NULL, x, dst, 0};
        parallel_for(M * N, q5_chunk, &J);
        return 0;
    }
    int isq8 = !strcmp(qtype, "q8"), isq4 = !strcmp(qtype, "q4");
    if (!isq8 && !isq4) return -1;
    if (G > 4096) return -1;
    int8_t *xq = malloc((size_t)M * K);
    float *xs = malloc((size_t)M * G * 4);
    int32_t *corr = malloc((size_t)M * G * 4);
    if (!xq || !xs || !corr) { free(xq); free(xs); free(corr); return -1; }
    for (int r = 0; r < M; r++) ref_quantize_act_q8(x + (size_t)r * K, G, xq + (size_t)r * K, xs + (size_t)r * G);
    int vnni = isq8 && bl_has_vnni();
    for (size_t i = 0; i < (size_t)M * G; i++) {
        int32_t s = 0;
        for (int k = 0; k < 32; k++) s += xq[i * 32 + k];
        corr[i] = (isq8 ? 128 : 8) * s;
    }
    job_t J = {raw, N, G, M, K, xq, xs, corr, x, dst, vnni};
    if (isq8) parallel_for(N, q8_chunk, &J);   /* parallelOverItems(outFeatures, ...) */
    else parallel_for(M * N, q4_chunk, &J);    /* parallelFor(xRows*outFeatures, ...) */
    free(xq); free(xs); free(corr);
    return 0;
}

/* Min over `trials` of the mean time of `reps` back-to-back matmuls (q8q8.go:280-294). */
double bl_time_matmul(const char *qtype, const uint8_t *raw, int N, int K, const float *x, int M,
                      float *dst, int reps, int trials) {
    double best = 1e30;
    if (bl_matmul(qtype, raw, N, K, x, M, dst)) return -1.0;
    for (int t = 0; t < trials; t++) {
        double t0 = now_s();
        for (int r = 0; r < reps; r++) bl_matmul(qtype, raw, N, K, x, M, dst);
        double dt = (now_s() - t0) / reps;
        if (dt < best) best = dt;
    }
    return best;
}
