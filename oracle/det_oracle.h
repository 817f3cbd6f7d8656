/*
 * det_oracle.h -- CPU oracle for MIND's deterministic integer / Q16.16
 * linear-algebra intrinsics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the *checker*: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.
 * The product path (mind_amd/, libmind_det_hip.so) never links or calls it.
 *
 * Every function restates the reference algorithm in plain scalar C and cites
 * the reference file:line it follows (paths relative to star-ga/mind v0.10.2).
 * Pinning (what checks each function against something other than itself):
 *   det_or_gemm_i8      -> golden sha256 gemm-i8-64x64x64 (917d353b...) and the
 *                          matmul_det_bench 256^3 digest words; brute force.
 *   det_or_gemm_q16     -> golden sha256 gemm-q16-64x64x64 (92e2cb75...);
 *                          closed form (S-R)>>16 computed with exact Python ints.
 *   det_or_gemv_q16     -> golden sha256 gemv-q16-256x256 (dfdf8908...); the
 *                          reference's own __mind_blas_dot_q16 (oracle/_ref).
 *   det_or_dot_q16      -> the reference's own __mind_blas_dot_q16 (oracle/_ref),
 *                          golden dot-l2-q16 (1d7f272b...).
 *   det_or_gemv_i16     -> golden sha256 gemv-i16-256x256 (3238e8c7...).
 *   det_or_dot_i16      -> golden dot-i16-4096 (af0fc3cf...).
 *   det_or_dot_l1_q16   -> golden dot-l1-q16 (ce7e2a80...); the reference's own
 *                          __mind_blas_dot_l1_q16 (oracle/_ref); exact Python-int
 *                          brute force incl. the |INT32_MIN - INT32_MAX| extreme.
 *   det_or_gemm_i16     -> composition: every element equals det_or_dot_i16 of
 *                          (row of A, column of B); exact Python-int brute force.
 *   det_or_dot_f32,     -> golden dot-f32-v-4093 (a132f7b9...) and
 *   det_or_matmul_rmajor_f32  matmul-f32-v-64x64 (ec5adb99...); the reference's
 *                          own __mind_blas_dot_f32 / __mind_blas_matmul_rmajor_f32
 *                          on both of its dispatch paths (oracle/_ref).
 *   det_or_dot_l1_f32,  -> the reference's own __mind_blas_dot_l1_f32 /
 *   det_or_dot_linf_f32    __mind_blas_dot_linf_f32 on both dispatch paths
 *                          (oracle/_ref; outputs in tests/golden/
 *                          dot_f32_metric_ref.json); exact closed forms (L-inf
 *                          = numpy max |a - b|, L1 of equal vectors = 0,
 *                          L1 of one block of 8 = the lane fold).
 *   det_or_dot_linf_f32_v -> the Track A max where no difference is NaN (the
 *                          reference's own lowering, lowering.rs:6219-6401,
 *                          is MLIR text that does not build here); NaN cases
 *                          pinned by the maximumf definition only.
 *   det_or_gen_*        -> the golden hashes above fix the reference draw order
 *                          and sample maps (next_i8 / next_i16 / next_q16).
 */
#ifndef DET_ORACLE_H
#define DET_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference LCG (benches/det_matmul_q16.rs:196-209) ---- */
uint32_t det_or_lcg_next_u32(uint64_t *state);

/* Draw all of `a` (na elements) then all of `b` (nb elements) from one LCG
 * stream seeded with `seed` (benches/det_matmul_i8.rs:221-226). */
void det_or_gen_i8(uint64_t seed, int8_t *a, int64_t na, int8_t *b, int64_t nb);
void det_or_gen_i16(uint64_t seed, int16_t *a, int64_t na, int16_t *b, int64_t nb);
/* (int32)u32 >> shift: shift 12 is the reference next_q16 (+-8.0),
 * 13 is +-4.0, 15 is +-1.0. */
void det_or_gen_q16(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb);
/* Q16 GEMM config generator: value = (int32)u32 >> shift, then one extra draw
 * r; when r % 100 == 0 the value becomes +-(2^31-1) (sign = bit 31 of r). */
void det_or_gen_q16_sat(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb);
/* MLP activations: s = sum of 12 draws of (u32 >> 16);
 * x = clamp(floor((2s - 12*65535) / 4096), -127, 127)  (sigma = 32). */
void det_or_gen_i8_gauss(uint64_t seed, int8_t *x, int64_t n);
/* MLP weights: (int8)(u32 >> 16), redrawn while == -128. */
void det_or_gen_i8_sym127(uint64_t seed, int8_t *w, int64_t n);

/* ---- scalar oracles ---- */
/* C[i,j] = (i32) sum_k (i64)A[i,k]*(i64)B[k,j]   (benches/det_matmul_i8.rs:232-245) */
void det_or_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, int64_t m, int64_t k, int64_t n);
/* Same, only for the listed rows; C is nrows x n. */
void det_or_gemm_i8_rows(const int8_t *A, const int8_t *B, int32_t *C, int64_t m, int64_t k,
                         int64_t n, const int64_t *rows, int64_t nrows);
/* C[i,j] = (i32) sum_k ((i64)A[i,k]*(i64)B[k,j] >> 16)   (benches/det_matmul_q16.rs:227-240) */
void det_or_gemm_q16(const int32_t *A, const int32_t *B, int32_t *C, int64_t m, int64_t k, int64_t n);
void det_or_gemm_q16_rows(const int32_t *A, const int32_t *B, int32_t *C, int64_t m, int64_t k,
                          int64_t n, const int64_t *rows, int64_t nrows);
/* C[i,j] = (i32) sum_k (i64)A[i,k]*(i64)B[k,j], int16 operands: each element is
 * the reference int16 dot (benches/det_matmul_i16.rs:218-224) of row i of A and
 * column j of B. */
void det_or_gemm_i16(const int16_t *A, const int16_t *B, int32_t *C, int64_t m, int64_t k, int64_t n);
void det_or_gemm_i16_rows(const int16_t *A, const int16_t *B, int32_t *C, int64_t m, int64_t k,
                          int64_t n, const int64_t *rows, int64_t nrows);
/* y[i] = (i32) sum_k ((i64)W[i,k]*(i64)x[k] >> 16)   (benches/det_gemv_q16_mt.rs:186-197) */
void det_or_gemv_q16(const int32_t *W, const int32_t *x, int32_t *y, int64_t m, int64_t k);
/* nb independent GEMVs: X is [nb][k], Y is [nb][m]. */
void det_or_gemv_q16_batched(const int32_t *W, const int32_t *X, int32_t *Y, int64_t m, int64_t k,
                             int64_t nb);
void det_or_gemv_q16_rows(const int32_t *W, const int32_t *X, int32_t *Y, int64_t m, int64_t k,
                          int64_t nb, const int64_t *rows, int64_t nrows);
/* y[r] = (i32) sum_i (i64)W[r,i]*(i64)x[i]   (benches/det_matmul_i16.rs:218-230) */
void det_or_gemv_i16(const int16_t *W, const int16_t *x, int32_t *y, int64_t rows, int64_t cols);
/* (i64)(i32) sum_i ((i64)a[i]*b[i] >> 16); 0 for len<=0 or NULL
 * (runtime-support/mind_intrinsics.c:1459-1471, 1537-1539). */
int64_t det_or_dot_q16(const int32_t *a, const int32_t *b, int64_t len);
/* (i64)(i32) sum_i (i64)a[i]*b[i]   (benches/det_matmul_i16.rs:218-224) */
int64_t det_or_dot_i16(const int16_t *a, const int16_t *b, int64_t len);
/* (int64)(int32) sum |a - b| in int64 (runtime-support/mind_intrinsics.c:
 * 1551-1562); len <= 0 or NULL -> 0 (:1598-1600). */
int64_t det_or_dot_l1_q16(const int32_t *a, const int32_t *b, int64_t len);

/* ---- strict-FP f32 (runtime-support/mind_intrinsics.c:1190-1290, 1418-1444;
 * src/mlir/lowering.rs emit_vec_dot_f32 :5528-5690).  Compiled with
 * -ffp-contract=off: every product is rounded before its add. ---- */
/* Lane j (0..7) sums a[i+j]*b[i+j] over full blocks of 8 in increasing i;
 * the 8 lanes are folded left to right, then the len % 8 tail is added in
 * order.  len <= 0 or NULL -> 0.0f. */
float det_or_dot_f32(const float *a, const float *b, int64_t len);
/* y[r] = det_or_dot_f32(W + r*cols, x, cols). */
void det_or_matmul_rmajor_f32(const float *W, const float *x, float *y, int64_t rows, int64_t cols);
/* f32 distances, results as their f32 bits (len <= 0 or NULL -> 0):
 * L1 = sum |a - b| on the dot's 8-lane schedule (sign-bit |x|);
 * L-infinity Track A = max over the non-NaN |a - b| (NaN skipped);
 * L-infinity vector twin = the same max, or 0x7fc00000 if any |a - b| is NaN. */
uint32_t det_or_dot_l1_f32(const float *a, const float *b, int64_t len);
uint32_t det_or_dot_linf_f32(const float *a, const float *b, int64_t len);
uint32_t det_or_dot_linf_f32_v(const float *a, const float *b, int64_t len);
/* y[r] = op(W row r, x) as bits: op 0 dot, 1 L1, 2 L-inf, 3 L-inf vector twin. */
void det_or_rows_metric_f32(int op, const float *W, const float *x, uint32_t *y, int64_t rows, int64_t cols);
/* f32 samples in [-1, 1): ((float)u32 / (float)UINT32_MAX) * 2 - 1, a then b
 * (tests/cross_substrate_identity.rs:2579-2598). */
void det_or_gen_f32_unit(uint64_t seed, float *a, int64_t na, float *b, int64_t nb);

/* ---- Q16.16 radix-2 DIT FFT (examples/fft_q16.mind, the fft256 symbol of
 * benches/fft_q16.rs; bench/fft/fft_ref.c is the same algorithm with the
 * span-2 stage unpeeled).  In place, n = 2^logn; returns -1 for any other
 * (logn, n).  Wrapping int64, qmul = low64(a*b) >> 16. ---- */
int64_t det_or_fft_q16(int64_t *re, int64_t *im, const int64_t *tw, int64_t logn, int64_t n);
void det_or_fft_twiddles(int64_t *tw, int64_t n);
void det_or_fft_input_lcg(uint64_t seed, int64_t *re, int64_t *im, int64_t n);
void det_or_fft_input_harness(uint64_t seed, int64_t *re, int64_t *im, int64_t n);
uint64_t det_or_fnv1a_i64(const int64_t *a, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
