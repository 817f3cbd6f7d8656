/*
 * det_oracle.c -- scalar CPU restatement of MIND's deterministic integer and
 * Q16.16 GEMM / GEMV intrinsics.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the product.
 * See det_oracle.h for what pins each function.
 *
 * Deliberately naive: one i64 accumulator per output element, k ascending,
 * exactly the loop the reference benches use as their own "independent scalar
 * oracle".  Arithmetic right shift of a negative int64 is relied on (gcc and
 * clang implement it as sign-propagating, as the reference C does too:
 * runtime-support/mind_intrinsics.c:1465-1469).
 */
#include "det_oracle.h"

#include <math.h>
#include <stddef.h>
#include <string.h>

/* benches/det_matmul_q16.rs:196-205:  s <- s*1664525 + 1013904223 (mod 2^64);
 * sample = (u32)(s >> 16). */
uint32_t det_or_lcg_next_u32(uint64_t *state) {
    *state = *state * 1664525ull + 1013904223ull;
    return (uint32_t)(*state >> 16);
}

/* benches/det_matmul_i8.rs:221-226: (i8)(u32 >> 16), A drawn before B. */
void det_or_gen_i8(uint64_t seed, int8_t *a, int64_t na, int8_t *b, int64_t nb) {
    uint64_t s = seed;
    for (int64_t i = 0; i < na; ++i) a[i] = (int8_t)(det_or_lcg_next_u32(&s) >> 16);
    for (int64_t i = 0; i < nb; ++i) b[i] = (int8_t)(det_or_lcg_next_u32(&s) >> 16);
}

/* benches/det_matmul_i16.rs:194-208: (i16)(u32 >> 16), W drawn before x. */
void det_or_gen_i16(uint64_t seed, int16_t *a, int64_t na, int16_t *b, int64_t nb) {
    uint64_t s = seed;
    for (int64_t i = 0; i < na; ++i) a[i] = (int16_t)(det_or_lcg_next_u32(&s) >> 16);
    for (int64_t i = 0; i < nb; ++i) b[i] = (int16_t)(det_or_lcg_next_u32(&s) >> 16);
}

/* benches/det_matmul_q16.rs:206-208 (shift 12) and its range variants. */
void det_or_gen_q16(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb) {
    uint64_t s = seed;
    for (int64_t i = 0; i < na; ++i) a[i] = ((int32_t)det_or_lcg_next_u32(&s)) >> shift;
    for (int64_t i = 0; i < nb; ++i) b[i] = ((int32_t)det_or_lcg_next_u32(&s)) >> shift;
}

static int32_t q16_sat_draw(uint64_t *s, int shift) {
    int32_t v = ((int32_t)det_or_lcg_next_u32(s)) >> shift;
    uint32_t r = det_or_lcg_next_u32(s);
    if (r % 100u == 0u) v = (r >> 31) ? -2147483647 : 2147483647;
    return v;
}

void det_or_gen_q16_sat(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb) {
    uint64_t s = seed;
    for (int64_t i = 0; i < na; ++i) a[i] = q16_sat_draw(&s, shift);
    for (int64_t i = 0; i < nb; ++i) b[i] = q16_sat_draw(&s, shift);
}

void det_or_gen_i8_gauss(uint64_t seed, int8_t *x, int64_t n) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) {
        int64_t acc = 0;
        for (int j = 0; j < 12; ++j) acc += (int64_t)(det_or_lcg_next_u32(&s) >> 16);
        int64_t t = 2 * acc - 12 * 65535;
        /* floor division by 4096 (t*32/131072) */
        int64_t q = t >= 0 ? t / 4096 : -((-t + 4095) / 4096);
        if (q > 127) q = 127;
        if (q < -127) q = -127;
        x[i] = (int8_t)q;
    }
}

void det_or_gen_i8_sym127(uint64_t seed, int8_t *w, int64_t n) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) {
        int8_t v;
        do {
            v = (int8_t)(det_or_lcg_next_u32(&s) >> 16);
        } while (v == -128);
        w[i] = v;
    }
}

/* ---------------------------------------------------------------- int8 */

static void gemm_i8_row(const int8_t *A, const int8_t *B, int32_t *c, int64_t i, int64_t k, int64_t n) {
    for (int64_t j = 0; j < n; ++j) {
        int64_t acc = 0;
        for (int64_t kk = 0; kk < k; ++kk) acc += (int64_t)A[i * k + kk] * (int64_t)B[kk * n + j];
        c[j] = (int32_t)acc;
    }
}

void det_or_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i) gemm_i8_row(A, B, C + i * n, i, k, n);
}

void det_or_gemm_i8_rows(const int8_t *A, const int8_t *B, int32_t *C, int64_t m, int64_t k, int64_t n,
                         const int64_t *rows, int64_t nrows) {
    (void)m;
    for (int64_t r = 0; r < nrows; ++r) gemm_i8_row(A, B, C + r * n, rows[r], k, n);
}

/* ---------------------------------------------------------------- Q16.16 */

static void gemm_q16_row(const int32_t *A, const int32_t *B, int32_t *c, int64_t i, int64_t k, int64_t n) {
    for (int64_t j = 0; j < n; ++j) {
        int64_t acc = 0;
        for (int64_t kk = 0; kk < k; ++kk) acc += ((int64_t)A[i * k + kk] * (int64_t)B[kk * n + j]) >> 16;
        c[j] = (int32_t)acc;
    }
}

void det_or_gemm_q16(const int32_t *A, const int32_t *B, int32_t *C, int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i) gemm_q16_row(A, B, C + i * n, i, k, n);
}

void det_or_gemm_q16_rows(const int32_t *A, const int32_t *B, int32_t *C, int64_t m, int64_t k, int64_t n,
                          const int64_t *rows, int64_t nrows) {
    (void)m;
    for (int64_t r = 0; r < nrows; ++r) gemm_q16_row(A, B, C + r * n, rows[r], k, n);
}

/* ---------------------------------------------------------------- int16 */

static void gemm_i16_row(const int16_t *A, const int16_t *B, int32_t *c, int64_t i, int64_t k, int64_t n) {
    for (int64_t j = 0; j < n; ++j) {
        int64_t acc = 0;
        for (int64_t kk = 0; kk < k; ++kk) acc += (int64_t)A[i * k + kk] * (int64_t)B[kk * n + j];
        c[j] = (int32_t)acc;
    }
}

void det_or_gemm_i16(const int16_t *A, const int16_t *B, int32_t *C, int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i) gemm_i16_row(A, B, C + i * n, i, k, n);
}

void det_or_gemm_i16_rows(const int16_t *A, const int16_t *B, int32_t *C, int64_t m, int64_t k, int64_t n,
                          const int64_t *rows, int64_t nrows) {
    (void)m;
    for (int64_t r = 0; r < nrows; ++r) gemm_i16_row(A, B, C + r * n, rows[r], k, n);
}

/* ---------------------------------------------------------------- GEMV */

int64_t det_or_dot_q16(const int32_t *a, const int32_t *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0;
    int64_t acc = 0;
    for (int64_t i = 0; i < len; ++i) acc += ((int64_t)a[i] * (int64_t)b[i]) >> 16;
    return (int64_t)(int32_t)acc;
}

int64_t det_or_dot_i16(const int16_t *a, const int16_t *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0;
    int64_t acc = 0;
    for (int64_t i = 0; i < len; ++i) acc += (int64_t)a[i] * (int64_t)b[i];
    return (int64_t)(int32_t)acc;
}

int64_t det_or_dot_l1_q16(const int32_t *a, const int32_t *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0;
    int64_t acc = 0;
    for (int64_t i = 0; i < len; ++i) {
        int64_t d = (int64_t)a[i] - (int64_t)b[i];
        acc += d < 0 ? -d : d;
    }
    return (int64_t)(int32_t)acc;
}

float det_or_dot_f32(const float *a, const float *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0.0f;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int64_t i = 0;
    for (; i + 8 <= len; i += 8)
        for (int j = 0; j < 8; ++j) {
            const float p = a[i + j] * b[i + j];
            acc[j] = acc[j] + p;
        }
    float s = acc[0];
    for (int j = 1; j < 8; ++j) s = s + acc[j];
    for (; i < len; ++i) {
        const float p = a[i] * b[i];
        s = s + p;
    }
    return s;
}

void det_or_matmul_rmajor_f32(const float *W, const float *x, float *y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) y[r] = det_or_dot_f32(W + r * cols, x, cols);
}

/* |x| by clearing the sign bit (runtime-support/mind_intrinsics.c:1210-1217,
 * the scalar twin of the AVX2 and-mask): -0.0 -> +0.0, NaN keeps its payload. */
static float or_abs_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u &= 0x7fffffffu;
    memcpy(&x, &u, 4);
    return x;
}

static uint32_t or_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

/* L1: mind_intrinsics.c:1293-1308 (scalar) -- the dot's 8-lane schedule with
 * |a - b| for the product: lane j sums positions j, j+8, ... in order, the
 * lanes fold left to right, then the len % 8 tail in order. */
uint32_t det_or_dot_l1_f32(const float *a, const float *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    int64_t i = 0;
    for (; i + 8 <= len; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] = acc[j] + or_abs_bits(a[i + j] - b[i + j]);
    float s = acc[0];
    for (int j = 1; j < 8; ++j) s = s + acc[j];
    for (; i < len; ++i) s = s + or_abs_bits(a[i] - b[i]);
    return or_bits(s);
}

/* L-infinity, Track A: mind_intrinsics.c:1355-1365 (scalar) -- m = 0; for
 * each i: d = a - b, negated when d < 0, kept when d > m.  A NaN d fails both
 * comparisons and is skipped. */
uint32_t det_or_dot_linf_f32(const float *a, const float *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0;
    float m = 0.0f;
    for (int64_t i = 0; i < len; ++i) {
        float d = a[i] - b[i];
        if (d < 0.0f) d = -d;
        if (d > m) m = d;
    }
    return or_bits(m);
}

/* L-infinity, vector twin: src/mlir/lowering.rs:6219-6401
 * (emit_vec_dot_metric_f32, VecMetric::Linf) -- arith.maximumf over the
 * sign-masked differences from 0.0: IEEE 754-2019 maximum, so any NaN
 * difference makes the result NaN.  Which NaN the reference returns is not
 * fixed by its lowering; this returns the quiet NaN 0x7fc00000. */
uint32_t det_or_dot_linf_f32_v(const float *a, const float *b, int64_t len) {
    if (len <= 0 || a == NULL || b == NULL) return 0;
    float m = 0.0f;
    for (int64_t i = 0; i < len; ++i) {
        const float d = or_abs_bits(a[i] - b[i]);
        if (d != d) return 0x7fc00000u;
        if (d > m) m = d;
    }
    return or_bits(m);
}

/* Row-major batched form: y[r] = metric(W row r, x), op 0 = dot, 1 = L1,
 * 2 = L-infinity (Track A), 3 = L-infinity (vector twin); results as bits. */
void det_or_rows_metric_f32(int op, const float *W, const float *x, uint32_t *y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *w = W + r * cols;
        uint32_t v = 0;
        if (op == 0) v = or_bits(det_or_dot_f32(w, x, cols));
        else if (op == 1) v = det_or_dot_l1_f32(w, x, cols);
        else if (op == 2) v = det_or_dot_linf_f32(w, x, cols);
        else v = det_or_dot_linf_f32_v(w, x, cols);
        y[r] = v;
    }
}

void det_or_gen_f32_unit(uint64_t seed, float *a, int64_t na, float *b, int64_t nb) {
    uint64_t s = seed;
    for (int64_t i = 0; i < na; ++i) a[i] = ((float)det_or_lcg_next_u32(&s) / (float)UINT32_MAX) * 2.0f - 1.0f;
    for (int64_t i = 0; i < nb; ++i) b[i] = ((float)det_or_lcg_next_u32(&s) / (float)UINT32_MAX) * 2.0f - 1.0f;
}

void det_or_gemv_q16(const int32_t *W, const int32_t *x, int32_t *y, int64_t m, int64_t k) {
    for (int64_t i = 0; i < m; ++i) y[i] = (int32_t)det_or_dot_q16(W + i * k, x, k);
}

void det_or_gemv_q16_batched(const int32_t *W, const int32_t *X, int32_t *Y, int64_t m, int64_t k, int64_t nb) {
    for (int64_t b = 0; b < nb; ++b) det_or_gemv_q16(W, X + b * k, Y + b * m, m, k);
}

void det_or_gemv_q16_rows(const int32_t *W, const int32_t *X, int32_t *Y, int64_t m, int64_t k, int64_t nb,
                          const int64_t *rows, int64_t nrows) {
    (void)m;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t r = 0; r < nrows; ++r)
            Y[b * nrows + r] = (int32_t)det_or_dot_q16(W + rows[r] * k, X + b * k, k);
}

void det_or_gemv_i16(const int16_t *W, const int16_t *x, int32_t *y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r) y[r] = (int32_t)det_or_dot_i16(W + r * cols, x, cols);
}

/* ---------------------------------------------------------------- Q16 FFT */
/* Wrapping int64 arithmetic (MIND's i64 ops lower to plain LLVM add / sub /
 * mul, which wrap); qmul is the low 64 bits of the product, then >> 16
 * arithmetic.  Follows examples/fft_q16.mind:15-120 (the fft256 symbol the
 * reference benches dlopen, benches/fft_q16.rs:66-168). */
static inline int64_t fft_add(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
static inline int64_t fft_sub(int64_t a, int64_t b) { return (int64_t)((uint64_t)a - (uint64_t)b); }
static inline int64_t fft_qmul(int64_t a, int64_t b) { return ((int64_t)((uint64_t)a * (uint64_t)b)) >> 16; }

int64_t det_or_fft_q16(int64_t *re, int64_t *im, const int64_t *tw, int64_t logn, int64_t n) {
    if (logn < 0 || logn > 30 || n != ((int64_t)1 << logn)) return -1;
    /* in-place bit-reversal permutation (fft_q16.mind:17-42) */
    for (int64_t i = 0; i < n; ++i) {
        int64_t r = 0;
        for (int64_t b = 0; b < logn; ++b) r |= ((i >> b) & 1) << (logn - 1 - b);
        if (r > i) {
            int64_t t = re[i]; re[i] = re[r]; re[r] = t;
            t = im[i]; im[i] = im[r]; im[r] = t;
        }
    }
    if (n < 2) return 0;
    /* span-2 stage, peeled: the kernel adds / subtracts without a twiddle
     * (fft_q16.mind:44-70) */
    for (int64_t a = 0; a < n; a += 2) {
        const int64_t ur = re[a], ui = im[a], xr = re[a + 1], xi = im[a + 1];
        re[a] = fft_add(ur, xr); im[a] = fft_add(ui, xi);
        re[a + 1] = fft_sub(ur, xr); im[a + 1] = fft_sub(ui, xi);
    }
    /* spans 4 .. n: butterfly (a, a + h) with twiddle index j * (n / span)
     * (fft_q16.mind:72-118) */
    for (int64_t span = 4; span <= n; span <<= 1) {
        const int64_t h = span >> 1, stride = n / span;
        for (int64_t base = 0; base < n; base += span)
            for (int64_t j = 0; j < h; ++j) {
                const int64_t wr = tw[2 * j * stride], wi = tw[2 * j * stride + 1];
                const int64_t a = base + j, b = a + h;
                const int64_t tr = fft_sub(fft_qmul(wr, re[b]), fft_qmul(wi, im[b]));
                const int64_t ti = fft_add(fft_qmul(wr, im[b]), fft_qmul(wi, re[b]));
                const int64_t ur = re[a], ui = im[a];
                re[a] = fft_add(ur, tr); im[a] = fft_add(ui, ti);
                re[b] = fft_sub(ur, tr); im[b] = fft_sub(ui, ti);
            }
    }
    return 0;
}

/* tw[2k] = llround(cos(-2 pi k / n) * 65536), tw[2k+1] = llround(sin(..) * 65536),
 * k < n / 2 (bench/fft/fft_driver.c:23-31, benches/fft_q16.rs:277-286). */
void det_or_fft_twiddles(int64_t *tw, int64_t n) {
    for (int64_t k = 0; k < n / 2; ++k) {
        const double ang = -2.0 * 3.14159265358979323846 * (double)k / (double)n;
        tw[2 * k] = (int64_t)llround(cos(ang) * 65536.0);
        tw[2 * k + 1] = (int64_t)llround(sin(ang) * 65536.0);
    }
}

/* The Rust / driver signal: re then im, (i64)((i32)u32 >> 13) from the
 * bench LCG (bench/fft/fft_driver.c:33-37, benches/fft_q16.rs:288-294). */
void det_or_fft_input_lcg(uint64_t seed, int64_t *re, int64_t *im, int64_t n) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) re[i] = (int64_t)(((int32_t)det_or_lcg_next_u32(&s)) >> 13);
    for (int64_t i = 0; i < n; ++i) im[i] = (int64_t)(((int32_t)det_or_lcg_next_u32(&s)) >> 13);
}

/* The harness.c signal (bench/fft/harness.c:50-53, 73-78): a 64-bit LCG
 * (6364136223846793005, 1442695040888963407), re[i] then im[i] interleaved
 * per i, sample (state mod 131072) - 65536. */
void det_or_fft_input_harness(uint64_t seed, int64_t *re, int64_t *im, int64_t n) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        re[i] = (int64_t)(s % 131072) - 65536;
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        im[i] = (int64_t)(s % 131072) - 65536;
    }
}

/* FNV-1a 64 over the little-endian bytes of n int64 (harness.c:40-45). */
uint64_t det_or_fnv1a_i64(const int64_t *a, int64_t n) {
    uint64_t h = 1469598103934665603ULL;
    const unsigned char *p = (const unsigned char *)a;
    for (int64_t i = 0; i < n * 8; ++i) { h ^= p[i]; h *= 1099511628211ULL; }
    return h;
}
