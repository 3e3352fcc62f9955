/*
 * cpu_baseline.c — the reference's per-call CPU arithmetic, for timing.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by bench.py's cpu_baseline leg (and the
 * oracle tests), never by the product.  The reference dequantizes weights to
 * f32 once at load time (barq_core/src/gguf.rs:437-475) and transposes the
 * projections (models/src/weight_cache.rs:172-210); per call it runs an f32
 * GEMM/GEMV.  Three variants are restated:
 *   (i)   literal:  blas::gemm_f32 CPU fallback at M=1 (blas.rs:199-210) —
 *         y[j] = sum_kk x[kk] * w_t[kk*n + j], the column-strided walk the
 *         decode loop runs on one core (rayon splits over M only);
 *   (ii)  SIMD:     the reference's AVX-512 dot (simd.rs:115-138; AVX2
 *         simd.rs:142-168 where AVX-512 is absent) per output row over the
 *         row-major dequantized weight, one thread;
 *   (iii) SIMD, all host threads: (ii) row-partitioned over pthreads.
 * For the batched configs:
 *   C4:   blas::gemm_f32 at M = 512 (blas.rs:193-212): output rows split over
 *         the host cores (rayon par_chunks_mut over rows of C), each row's
 *         columns in order, kk sequential over the column-strided W^T;
 *   C5:   MoEFusedOps::dispatch_experts (moe_fused.rs:226-308) with each
 *         expert's fused_ffn (:84-92): ops::MatMul (ops.rs:68-128, one
 *         thread, the same sequential sum) for x G and x U, ops::Silu
 *         x / (1 + exp(-x)) (:191-211) times x U, MatMul with D, over f32
 *         weights transposed at load.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>

/* (i) blas.rs:199-210 for i = 0, columns [j0, j1) */
void cpub_gemm_literal_m1(const float* x, const float* w_t, size_t k, size_t n,
                          size_t j0, size_t j1, float* y) {
    for (size_t j = j0; j < j1; j++) {
        float sum = 0.0f;
        for (size_t kk = 0; kk < k; kk++) sum += x[kk] * w_t[kk * n + j];
        y[j] = sum;
    }
}

__attribute__((target("avx512f")))
static float dot_avx512(const float* a, const float* b, size_t len) {
    __m512 sum = _mm512_setzero_ps();
    size_t i = 0;
    for (; i + 16 <= len; i += 16)
        sum = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), sum);
    float lanes[16];
    _mm512_storeu_ps(lanes, sum);
    float total = 0.0f;
    for (int l = 0; l < 16; l++) total += lanes[l];
    for (; i < len; i++) total += a[i] * b[i];
    return total;
}

__attribute__((target("avx2,fma")))
static float dot_avx2(const float* a, const float* b, size_t len) {
    __m256 sum = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= len; i += 8)
        sum = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), sum);
    float lanes[8];
    _mm256_storeu_ps(lanes, sum);
    float total = 0.0f;
    for (int l = 0; l < 8; l++) total += lanes[l];
    for (; i < len; i++) total += a[i] * b[i];
    return total;
}

/* 2 = AVX-512, 1 = AVX2, 0 = scalar */
int cpub_simd_level(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f")) return 2;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 1;
    return 0;
}

static float dot_any(int level, const float* a, const float* b, size_t len) {
    if (level == 2) return dot_avx512(a, b, len);
    if (level == 1) return dot_avx2(a, b, len);
    float s = 0.0f;
    for (size_t i = 0; i < len; i++) s += a[i] * b[i];
    return s;
}

/* (ii) rows [r0, r1) of y = A x with the reference SIMD dot */
void cpub_gemv_simd(const float* a, const float* x, size_t n, size_t r0, size_t r1, float* y) {
    int level = cpub_simd_level();
    for (size_t r = r0; r < r1; r++) y[r] = dot_any(level, a + r * n, x, n);
}

struct job { const float* a; const float* x; size_t n, r0, r1; float* y; };

static void* run_job(void* p) {
    struct job* j = (struct job*)p;
    cpub_gemv_simd(j->a, j->x, j->n, j->r0, j->r1, j->y);
    return NULL;
}

/* (iii) rows [r0, r1) split over `threads` pthreads (at most 512); returns
   the number of row ranges run (a range whose thread cannot be created runs
   on the calling thread) */
#define CPUB_MAX_THREADS 512
int cpub_gemv_simd_threaded(const float* a, const float* x, size_t n, size_t r0, size_t r1,
                            float* y, int threads) {
    if (threads < 1) threads = 1;
    if (threads > CPUB_MAX_THREADS) threads = CPUB_MAX_THREADS;
    pthread_t tid[CPUB_MAX_THREADS];
    char created[CPUB_MAX_THREADS];
    struct job jobs[CPUB_MAX_THREADS];
    size_t rows = r1 - r0, per = (rows + (size_t)threads - 1) / (size_t)threads;
    int used = 0;
    for (int t = 0; t < threads; t++) {
        size_t s = r0 + (size_t)t * per, e = s + per < r1 ? s + per : r1;
        if (s >= e) break;
        jobs[t] = (struct job){a, x, n, s, e, y};
        created[t] = pthread_create(&tid[t], NULL, run_job, &jobs[t]) == 0;
        if (!created[t]) run_job(&jobs[t]);
        used = t + 1;
    }
    for (int t = 0; t < used; t++)
        if (created[t]) pthread_join(tid[t], NULL);
    return used;
}

/* blas.rs:202-210 / ops.rs:95-106: rows [i0, i1) of C[m x n] = A[m x k] B[k x n],
   each element a sequential unfused sum over kk */
void cpub_gemm_rows(const float* a, const float* b, size_t k, size_t n, size_t i0, size_t i1, float* c) {
    for (size_t i = i0; i < i1; i++)
        for (size_t j = 0; j < n; j++) {
            float sum = 0.0f;
            for (size_t kk = 0; kk < k; kk++) sum += a[i * k + kk] * b[kk * n + j];
            c[i * n + j] = sum;
        }
}

struct gjob { const float* a; const float* b; size_t k, n, i0, i1; float* c; };

static void* run_gjob(void* p) {
    struct gjob* j = (struct gjob*)p;
    cpub_gemm_rows(j->a, j->b, j->k, j->n, j->i0, j->i1, j->c);
    return NULL;
}

/* gemm_f32's rayon form: rows [i0, i1) split over `threads` pthreads
   (returns the number of row ranges run) */
int cpub_gemm_rows_threaded(const float* a, const float* b, size_t k, size_t n, size_t i0, size_t i1, float* c,
                            int threads) {
    if (threads < 1) threads = 1;
    if (threads > CPUB_MAX_THREADS) threads = CPUB_MAX_THREADS;
    pthread_t tid[CPUB_MAX_THREADS];
    char created[CPUB_MAX_THREADS];
    struct gjob jobs[CPUB_MAX_THREADS];
    size_t rows = i1 - i0, per = (rows + (size_t)threads - 1) / (size_t)threads;
    int used = 0;
    for (int t = 0; t < threads; t++) {
        size_t s = i0 + (size_t)t * per, e = s + per < i1 ? s + per : i1;
        if (s >= e) break;
        jobs[t] = (struct gjob){a, b, k, n, s, e, c};
        created[t] = pthread_create(&tid[t], NULL, run_gjob, &jobs[t]) == 0;
        if (!created[t]) run_gjob(&jobs[t]);
        used = t + 1;
    }
    for (int t = 0; t < used; t++)
        if (created[t]) pthread_join(tid[t], NULL);
    return used;
}

/* fused_ffn of one expert on t rows (moe_fused.rs:84-92): g = x Gt, u = x Ut
   (Gt, Ut [hidden x n_ff]), h = (g / (1 + exp(-g))) * u, out = h Dt
   (Dt [n_ff x hidden]); g and u are t x n_ff scratch */
void cpub_moe_expert_ffn(const float* x, size_t t, size_t hidden, size_t n_ff, const float* gt, const float* ut,
                         const float* dt, float* g, float* u, float* out) {
    cpub_gemm_rows(x, gt, hidden, n_ff, 0, t, g);
    cpub_gemm_rows(x, ut, hidden, n_ff, 0, t, u);
    for (size_t i = 0; i < t * n_ff; i++) {
        const float a = g[i] / (1.0f + expf(-g[i]));
        g[i] = a * u[i];
    }
    cpub_gemm_rows(g, dt, n_ff, hidden, 0, t, out);
}
