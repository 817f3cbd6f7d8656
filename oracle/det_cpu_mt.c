/*
 * det_cpu_mt.c -- multithreaded CPU restatement of the reference's MT
 * deterministic GEMM / GEMV path, used as the *reported CPU baseline*.
 *
 * TEST INFRASTRUCTURE ONLY (cpu_baseline leg of bench.py and tests).  It is a
 * restatement ("port"), not the reference build: the reference kernels are
 * MLIR text emitted by Rust (src/mlir/lowering.rs) and need cargo + mlir-opt,
 * which this image does not have.
 *
 * What it restates:
 *   - owner-computes M-row bands, T = clamp(online CPUs, 1, min(M, 256)),
 *     band = ceil(M / T)            (src/mlir/lowering.rs:10146-10190)
 *   - a persistent worker pool created lazily once, a dispatch lock that
 *     serialises callers, condvar wake / join
 *                                   (runtime-support/mind_intrinsics.c:1935-2082)
 *   - per band, the BLIS loop nest jc -> ic -> pc -> jr -> ir with packed
 *     A/B panels and a C-scratch truncated to i32 once at the store
 *                                   (src/mlir/lowering.rs:7074-7676, 8371-9265)
 *   - tile constants                (src/mlir/gemm_tuning.rs:61-159)
 *       int8: MC/KC/NC = 1024/512/128, MR x NR = 4 x 16
 *       Q16 : MC/KC/NC =   64/256/128, MR x NR = 4 x 8
 *   - the AVX2 microkernels, written with intrinsics in the shape the
 *     reference emits them:
 *       int8 (lowering.rs:7798-8052): panels packed to i16 K-pairs; per K
 *       pair the NR/8 = 2 B vectors are loaded once, each row's A pair is
 *       broadcast as one i32 and contracted with both by vpmaddwd into i32
 *       accumulators (vpaddd), 4 x 2 ymm accumulators, an i32 C-scratch;
 *       Q16 (lowering.rs:7470-7540): per k the 8 B values are sign-extended
 *       to i64, each row's A value broadcast, multiplied (vpmuldq), shifted
 *       arithmetically by 16 and added into 4 x 2 ymm i64 accumulators;
 *   - GEMV: one row band per worker, per-row Q16 dot 8 lanes wide in i64
 *     (vpmuldq + shift + add), a scalar K % 8 tail, lane sums folded at the
 *     end                           (src/mlir/lowering.rs:9822-9997)
 * Built with -O3 -march=x86-64-v3 -ffp-contract=off -pthread, the flags the
 * reference passes to clang (src/eval/mlir_build.rs:685-760).
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define POOL_MAX 256

typedef void (*band_fn)(void *);

static struct {
    pthread_mutex_t mtx;
    pthread_cond_t wake, done;
    band_fn fn;
    char *args;
    long stride, active, finished, gen, pool_n;
    pthread_t th[POOL_MAX];
} pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER};

static pthread_mutex_t dispatch_lock = PTHREAD_MUTEX_INITIALIZER;
static long thread_override = 0;

static void *worker_loop(void *p) {
    long id = (long)(intptr_t)p, seen = 0;
    for (;;) {
        pthread_mutex_lock(&pool.mtx);
        while (pool.gen == seen) pthread_cond_wait(&pool.wake, &pool.mtx);
        seen = pool.gen;
        int mine = id < pool.active;
        band_fn fn = pool.fn;
        void *arg = mine ? pool.args + id * pool.stride : NULL;
        pthread_mutex_unlock(&pool.mtx);
        if (mine) {
            fn(arg);
            pthread_mutex_lock(&pool.mtx);
            pool.finished++;
            pthread_cond_signal(&pool.done);
            pthread_mutex_unlock(&pool.mtx);
        }
    }
    return NULL;
}

static void pool_init(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > POOL_MAX) n = POOL_MAX;
    pool.pool_n = n;
    for (long i = 0; i < n; ++i) {
        pthread_attr_t at;
        pthread_attr_init(&at);
        pthread_attr_setdetachstate(&at, PTHREAD_CREATE_DETACHED);
        pthread_create(&pool.th[i], &at, worker_loop, (void *)(intptr_t)i);
        pthread_attr_destroy(&at);
    }
}

static void dispatch(band_fn fn, void *args, long stride, long nbands) {
    static pthread_once_t once = PTHREAD_ONCE_INIT;
    if (nbands <= 0) return;
    pthread_once(&once, pool_init);
    if (nbands > pool.pool_n) nbands = pool.pool_n;
    pthread_mutex_lock(&dispatch_lock);
    pthread_mutex_lock(&pool.mtx);
    pool.fn = fn;
    pool.args = (char *)args;
    pool.stride = stride;
    pool.active = nbands;
    pool.finished = 0;
    pool.gen++;
    pthread_cond_broadcast(&pool.wake);
    while (pool.finished < nbands) pthread_cond_wait(&pool.done, &pool.mtx);
    pthread_mutex_unlock(&pool.mtx);
    pthread_mutex_unlock(&dispatch_lock);
}

/* Number of bands T for M rows (src/mlir/lowering.rs:10146-10190). */
static long band_count(int64_t m) {
    long t = thread_override > 0 ? thread_override : sysconf(_SC_NPROCESSORS_ONLN);
    if (t < 1) t = 1;
    if (t > POOL_MAX) t = POOL_MAX;
    if (t > m) t = (long)m;
    return t;
}

/* Force the band count (0 restores the CPU count); returns the CPU count. */
long det_cpu_set_threads(long t) {
    thread_override = t;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n < 1 ? 1 : n;
}

long det_cpu_threads_for(int64_t m) { return band_count(m); }

typedef struct {
    const void *a, *b;
    void *c;
    int64_t k, n, m, r0, r1;
} band_args;

static long make_bands(band_args *args, const void *a, const void *b, void *c, int64_t m, int64_t k, int64_t n) {
    long t = band_count(m);
    int64_t band = (m + t - 1) / t;
    long nb = 0;
    for (long i = 0; i < t; ++i) {
        int64_t r0 = i * band, r1 = r0 + band < m ? r0 + band : m;
        if (r0 >= r1) break;
        band_args ba = {a, b, c, k, n, m, r0, r1};
        args[nb++] = ba;
    }
    return nb;
}

/* ----------------------------------------------------------- int8 band */

#define I8_MC 1024
#define I8_KC 512
#define I8_NC 128
#define I8_MR 4
#define I8_NR 16

/* 4 x 16 int8 microkernel over kp K pairs: acc[r][g] holds columns 8g..8g+7
 * of row r.  bq: [kp][16 columns][2] i16, aq: [kp][4 rows][2] i16. */
static inline void i8_micro(const int16_t *aq, const int16_t *bq, int64_t kp, int32_t *cs, int64_t ldc) {
    __m256i acc[I8_MR][2];
    for (int r = 0; r < I8_MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_si256();
    for (int64_t q = 0; q < kp; ++q) {
        const __m256i b0 = _mm256_load_si256((const __m256i *)(bq + q * 2 * I8_NR));
        const __m256i b1 = _mm256_load_si256((const __m256i *)(bq + q * 2 * I8_NR + 16));
        const int16_t *a = aq + q * 2 * I8_MR;
        for (int r = 0; r < I8_MR; ++r) {
            int32_t pair;
            memcpy(&pair, a + 2 * r, 4);
            const __m256i av = _mm256_set1_epi32(pair);   /* [a0, a1] in every 32-bit lane */
            acc[r][0] = _mm256_add_epi32(acc[r][0], _mm256_madd_epi16(av, b0));
            acc[r][1] = _mm256_add_epi32(acc[r][1], _mm256_madd_epi16(av, b1));
        }
    }
    for (int r = 0; r < I8_MR; ++r)
        for (int g = 0; g < 2; ++g) {
            __m256i *c = (__m256i *)(cs + r * ldc + 8 * g);
            _mm256_storeu_si256(c, _mm256_add_epi32(_mm256_loadu_si256(c), acc[r][g]));
        }
}

static void i8_band(void *p) {
    band_args *ba = (band_args *)p;
    const int8_t *A = (const int8_t *)ba->a, *B = (const int8_t *)ba->b;
    int32_t *C = (int32_t *)ba->c;
    const int64_t k = ba->k, n = ba->n;
    /* packed panels are i16 (sign-extended once at pack time), K-pair
     * interleaved like the vpmaddwd microkernel consumes them; the C-scratch
     * is i32 (the AVX2 rung's: i32 partials end to end, wrapped like the
     * final truncation) */
    int16_t *bp = (int16_t *)aligned_alloc(64, sizeof(int16_t) * (I8_KC + 2) * I8_NC);
    int16_t *ap = (int16_t *)aligned_alloc(64, sizeof(int16_t) * (I8_KC + 2) * I8_MC);
    int32_t *cs = (int32_t *)aligned_alloc(64, sizeof(int32_t) * I8_MC * I8_NC);
    for (int64_t jc = 0; jc < n; jc += I8_NC) {
        const int64_t nc = n - jc < I8_NC ? n - jc : I8_NC;
        const int64_t ncp = (nc + I8_NR - 1) / I8_NR * I8_NR;
        for (int64_t ic = ba->r0; ic < ba->r1; ic += I8_MC) {
            const int64_t mc = ba->r1 - ic < I8_MC ? ba->r1 - ic : I8_MC;
            const int64_t mcp = (mc + I8_MR - 1) / I8_MR * I8_MR;
            memset(cs, 0, sizeof(int32_t) * mcp * ncp);
            for (int64_t pc = 0; pc < k; pc += I8_KC) {
                const int64_t kc = k - pc < I8_KC ? k - pc : I8_KC;
                const int64_t kp = (kc + 1) / 2; /* K pairs, zero padded */
                /* pack B: [jr block][kpair][NR][2] */
                for (int64_t jr = 0; jr < ncp; jr += I8_NR) {
                    int16_t *d = bp + (jr / I8_NR) * kp * 2 * I8_NR;
                    for (int64_t q = 0; q < kp; ++q)
                        for (int e = 0; e < 2; ++e) {
                            const int64_t kk = 2 * q + e;
                            const int8_t *src = B + (pc + kk) * n + jc + jr;
                            for (int64_t c = 0; c < I8_NR; ++c)
                                d[q * 2 * I8_NR + 2 * c + e] = (kk < kc && jr + c < nc) ? src[c] : 0;
                        }
                }
                /* pack A: [ir block][kpair][MR][2] */
                for (int64_t ir = 0; ir < mcp; ir += I8_MR) {
                    int16_t *d = ap + (ir / I8_MR) * kp * 2 * I8_MR;
                    for (int64_t r = 0; r < I8_MR; ++r) {
                        const int8_t *src = A + (ic + ir + r) * k + pc;
                        const int ok = ir + r < mc;
                        for (int64_t kk = 0; kk < 2 * kp; ++kk)
                            d[(kk >> 1) * 2 * I8_MR + 2 * r + (kk & 1)] = (ok && kk < kc) ? src[kk] : 0;
                    }
                }
                for (int64_t jr = 0; jr < ncp; jr += I8_NR) {
                    const int16_t *bb = bp + (jr / I8_NR) * kp * 2 * I8_NR;
                    for (int64_t ir = 0; ir < mcp; ir += I8_MR)
                        i8_micro(ap + (ir / I8_MR) * kp * 2 * I8_MR, bb, kp, cs + ir * ncp + jr, ncp);
                }
            }
            for (int64_t i = 0; i < mc; ++i) memcpy(C + (ic + i) * n + jc, cs + i * ncp, sizeof(int32_t) * nc);
        }
    }
    free(bp);
    free(ap);
    free(cs);
}

/* ----------------------------------------------------------- Q16 band */

#define Q_MC 64
#define Q_KC 256
#define Q_NC 128
#define Q_MR 4
#define Q_NR 8

/* Arithmetic shift right by 16 of four i64 lanes (AVX2 has no vpsraq):
 * offset by 2^63, shift logically, remove the shifted offset. */
static inline __m256i sra16_epi64(__m256i x) {
    const __m256i bias = _mm256_set1_epi64x((long long)0x8000000000000000ull);
    return _mm256_sub_epi64(_mm256_srli_epi64(_mm256_xor_si256(x, bias), 16), _mm256_srli_epi64(bias, 16));
}

/* 4 x 8 Q16 microkernel over kc k: acc[r][h] holds columns 4h..4h+3 of row r
 * as i64.  bq: [kc][8] i32, aq: [kc][4] i32. */
static inline void q16_micro(const int32_t *aq, const int32_t *bq, int64_t kc, int64_t *cs, int64_t ldc) {
    __m256i acc[Q_MR][2];
    for (int r = 0; r < Q_MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_si256();
    for (int64_t kk = 0; kk < kc; ++kk) {
        const __m256i bv = _mm256_load_si256((const __m256i *)(bq + kk * Q_NR));
        const __m256i b0 = _mm256_cvtepi32_epi64(_mm256_castsi256_si128(bv));
        const __m256i b1 = _mm256_cvtepi32_epi64(_mm256_extracti128_si256(bv, 1));
        for (int r = 0; r < Q_MR; ++r) {
            const __m256i av = _mm256_set1_epi64x((long long)aq[kk * Q_MR + r]);
            acc[r][0] = _mm256_add_epi64(acc[r][0], sra16_epi64(_mm256_mul_epi32(av, b0)));
            acc[r][1] = _mm256_add_epi64(acc[r][1], sra16_epi64(_mm256_mul_epi32(av, b1)));
        }
    }
    for (int r = 0; r < Q_MR; ++r)
        for (int h = 0; h < 2; ++h) {
            __m256i *c = (__m256i *)(cs + r * ldc + 4 * h);
            _mm256_storeu_si256(c, _mm256_add_epi64(_mm256_loadu_si256(c), acc[r][h]));
        }
}

static void q16_band(void *p) {
    band_args *ba = (band_args *)p;
    const int32_t *A = (const int32_t *)ba->a, *B = (const int32_t *)ba->b;
    int32_t *C = (int32_t *)ba->c;
    const int64_t k = ba->k, n = ba->n;
    /* packed panels (B: [jr block][kk][NR], A: [ir block][kk][MR]) and the
     * i64 C-scratch: the reference keeps them on the stack (alloca) */
    int32_t bp[Q_KC * Q_NC] __attribute__((aligned(64)));
    int32_t ap[Q_MC * Q_KC] __attribute__((aligned(64)));
    int64_t cs[Q_MC * Q_NC] __attribute__((aligned(64)));
    for (int64_t jc = 0; jc < n; jc += Q_NC) {
        const int64_t nc = n - jc < Q_NC ? n - jc : Q_NC;
        const int64_t ncp = (nc + Q_NR - 1) / Q_NR * Q_NR;
        for (int64_t ic = ba->r0; ic < ba->r1; ic += Q_MC) {
            const int64_t mc = ba->r1 - ic < Q_MC ? ba->r1 - ic : Q_MC;
            const int64_t mcp = (mc + Q_MR - 1) / Q_MR * Q_MR;
            memset(cs, 0, sizeof cs);
            for (int64_t pc = 0; pc < k; pc += Q_KC) {
                const int64_t kc = k - pc < Q_KC ? k - pc : Q_KC;
                for (int64_t jr = 0; jr < ncp; jr += Q_NR) {
                    int32_t *d = bp + (jr / Q_NR) * kc * Q_NR;
                    for (int64_t kk = 0; kk < kc; ++kk) {
                        const int32_t *src = B + (pc + kk) * n + jc + jr;
                        for (int64_t c = 0; c < Q_NR; ++c) d[kk * Q_NR + c] = jr + c < nc ? src[c] : 0;
                    }
                }
                for (int64_t ir = 0; ir < mcp; ir += Q_MR) {
                    int32_t *d = ap + (ir / Q_MR) * kc * Q_MR;
                    for (int64_t r = 0; r < Q_MR; ++r) {
                        const int32_t *src = A + (ic + ir + r) * k + pc;
                        const int ok = ir + r < mc;
                        for (int64_t kk = 0; kk < kc; ++kk) d[kk * Q_MR + r] = ok ? src[kk] : 0;
                    }
                }
                for (int64_t jr = 0; jr < ncp; jr += Q_NR)
                    for (int64_t ir = 0; ir < mcp; ir += Q_MR)
                        q16_micro(ap + (ir / Q_MR) * kc * Q_MR, bp + (jr / Q_NR) * kc * Q_NR, kc,
                                  cs + ir * Q_NC + jr, Q_NC);
            }
            for (int64_t i = 0; i < mc; ++i)
                for (int64_t j = 0; j < nc; ++j) C[(ic + i) * n + jc + j] = (int32_t)cs[i * Q_NC + j];
        }
    }
}

/* ----------------------------------------------------------- int16 band */

static void i16_band(void *p) {
    band_args *ba = (band_args *)p;
    const int16_t *A = (const int16_t *)ba->a, *B = (const int16_t *)ba->b;
    int32_t *C = (int32_t *)ba->c;
    const int64_t k = ba->k, n = ba->n;
    int64_t *row = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n > 0 ? n : 1));
    for (int64_t i = ba->r0; i < ba->r1; ++i) {
        memset(row, 0, sizeof(int64_t) * (size_t)n);
        for (int64_t kk = 0; kk < k; ++kk) {
            const int64_t a = A[i * k + kk];
            const int16_t *b = B + kk * n;
            for (int64_t j = 0; j < n; ++j) row[j] += a * (int64_t)b[j];
        }
        for (int64_t j = 0; j < n; ++j) C[i * n + j] = (int32_t)row[j];
    }
    free(row);
}

/* ----------------------------------------------------------- GEMV band */

static void gemv_q16_band(void *p) {
    band_args *ba = (band_args *)p;
    const int32_t *W = (const int32_t *)ba->a, *x = (const int32_t *)ba->b;
    int32_t *y = (int32_t *)ba->c;
    const int64_t k = ba->k, kmain = k / 8 * 8;
    for (int64_t i = ba->r0; i < ba->r1; ++i) {
        const int32_t *w = W + i * k;
        __m256i acc0 = _mm256_setzero_si256(), acc1 = _mm256_setzero_si256();
        for (int64_t kk = 0; kk < kmain; kk += 8) {
            const __m256i wv = _mm256_loadu_si256((const __m256i *)(w + kk));
            const __m256i xv = _mm256_loadu_si256((const __m256i *)(x + kk));
            const __m256i w0 = _mm256_cvtepi32_epi64(_mm256_castsi256_si128(wv));
            const __m256i w1 = _mm256_cvtepi32_epi64(_mm256_extracti128_si256(wv, 1));
            const __m256i x0 = _mm256_cvtepi32_epi64(_mm256_castsi256_si128(xv));
            const __m256i x1 = _mm256_cvtepi32_epi64(_mm256_extracti128_si256(xv, 1));
            acc0 = _mm256_add_epi64(acc0, sra16_epi64(_mm256_mul_epi32(w0, x0)));
            acc1 = _mm256_add_epi64(acc1, sra16_epi64(_mm256_mul_epi32(w1, x1)));
        }
        int64_t lanes[8];
        _mm256_storeu_si256((__m256i *)lanes, acc0);
        _mm256_storeu_si256((__m256i *)(lanes + 4), acc1);
        int64_t acc = 0;
        for (int l = 0; l < 8; ++l) acc += lanes[l];
        for (int64_t kk = kmain; kk < k; ++kk) acc += ((int64_t)w[kk] * (int64_t)x[kk]) >> 16;
        y[i] = (int32_t)acc;
    }
}

static void run(band_fn fn, const void *a, const void *b, void *c, int64_t m, int64_t k, int64_t n) {
    band_args args[POOL_MAX];
    long nb = make_bands(args, a, b, c, m, k, n);
    dispatch(fn, args, sizeof(band_args), nb);
}

int64_t det_cpu_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || n <= 0) return 0;
    run(i8_band, A, B, C, m, k, n);
    return 0;
}

int64_t det_cpu_gemm_q16(const int32_t *A, const int32_t *B, int32_t *C, int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || n <= 0) return 0;
    run(q16_band, A, B, C, m, k, n);
    return 0;
}

int64_t det_cpu_gemm_i16(const int16_t *A, const int16_t *B, int32_t *C, int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || n <= 0) return 0;
    run(i16_band, A, B, C, m, k, n);
    return 0;
}

int64_t det_cpu_gemv_q16(const int32_t *W, const int32_t *x, int32_t *y, int64_t m, int64_t k) {
    if (m <= 0) return 0;
    run(gemv_q16_band, W, x, y, m, k, 1);
    return 0;
}
