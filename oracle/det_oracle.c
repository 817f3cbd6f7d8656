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

#include <stddef.h>

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
