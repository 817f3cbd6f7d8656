/*
 * mind_det.h -- C ABI of libmind_det_hip.so: MIND's deterministic integer and
 * Q16.16 linear-algebra intrinsics as hand-written HIP kernels for MI355X
 * (gfx950).  Every result is bit-identical to the reference CPU kernels.
 *
 * Citations are into star-ga/mind v0.10.2.  Arithmetic contract:
 *   int8 GEMM : C[i,j] = (int32) sum_k A[i,k]*B[k,j]              (exact, wrapped)
 *   Q16 GEMM  : C[i,j] = (int32) sum_k ((int64)A[i,k]*B[k,j] >>arith 16)
 *   int16     : (int32) sum (int64)a*b                            (exact, wrapped)
 *   Q16 GEMV  : y[i]   = (int32) sum_k ((int64)W[i,k]*x[k] >>arith 16)
 * All matrices are dense row-major; B is K x N (not transposed) unless a
 * symbol says otherwise.
 *
 * Layer 1 and 2 keep the reference's i64 "Option C" ABI: every pointer is an
 * int64_t address of HOST memory, the call is synchronous, and it returns 0
 * on success.  A NULL pointer or an empty shape returns 0 and writes nothing
 * (Track A convention, runtime-support/mind_intrinsics.c:1537-1539).  A
 * negative return is a device failure or an invalid shape (dimension
 * outside [0, 2^31)); det_last_error() describes it.
 */
#ifndef MIND_DET_H
#define MIND_DET_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes (negative returns) */
#define DET_ERR_ARG (-22)
#define DET_ERR_HIP (-5)
#define DET_ERR_DEVICE (-19)

/* op selectors for the workspace-explicit entry points */
#define DET_OP_I8 1
#define DET_OP_I16 2
#define DET_OP_Q16 3
#define DET_DOT_Q16 0
#define DET_DOT_L1_Q16 1
#define DET_DOT_I16 2
/* f32 metrics of det_rows_metric_f32[_dev] */
#define DET_F32_DOT 0
#define DET_F32_L1 1
#define DET_F32_LINF 2
#define DET_F32_LINF_V 3

/* ------------------------------------------------------------------------
 * Layer 1: the reference's intrinsic symbols (arity table
 * src/type_checker/mod.rs:2266-2332).
 * ---------------------------------------------------------------------- */

/* Replaces __mind_blas_matmul_mm_i8_v: src/type_checker/mod.rs:2304,
 * src/mlir/lowering.rs:2918-2925 (dispatch), :7687-7797, :8371-9265. */
int64_t __mind_blas_matmul_mm_i8_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* Replaces __mind_blas_matmul_mm_i8_mt_v: src/mlir/lowering.rs:2935-2942,
 * :10368-10700 (owner-computes row bands; here one GPU grid). */
int64_t __mind_blas_matmul_mm_i8_mt_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* Replaces __mind_blas_matmul_mm_q16_v: src/type_checker/mod.rs:2316,
 * src/mlir/lowering.rs:2864-2871, :9300-9410. */
int64_t __mind_blas_matmul_mm_q16_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* Replaces __mind_blas_matmul_mm_q16_mt_v: src/mlir/lowering.rs:2879-2891,
 * :10019-10340. */
int64_t __mind_blas_matmul_mm_q16_mt_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* Replaces __mind_blas_gemv_q16_mt(w, x, y, m, k): src/type_checker/mod.rs:2332,
 * src/mlir/lowering.rs:2901-2907, :9822-9997. */
int64_t __mind_blas_gemv_q16_mt(int64_t w, int64_t x, int64_t y, int64_t m, int64_t k);
/* Replaces __mind_blas_matmul_rmajor_q16_v(w, x, y, rows, cols):
 * src/mlir/lowering.rs:2847-2852, :6675-7035. */
int64_t __mind_blas_matmul_rmajor_q16_v(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);
/* Replaces __mind_blas_matmul_rmajor_i16_v(w, x, y, rows, cols):
 * src/type_checker/mod.rs:2285, src/mlir/lowering.rs:2948-2953, :10723-11150. */
int64_t __mind_blas_matmul_rmajor_i16_v(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);
/* Replaces __mind_blas_dot_q16(a, b, len) -> (int64)(int32)sum:
 * runtime-support/mind_intrinsics.c:1537-1547.  Returns the value. */
int64_t __mind_blas_dot_q16(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_q16_v (the vector-dialect twin of the above):
 * src/mlir/lowering.rs:5695-5860. */
int64_t __mind_blas_dot_q16_v(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_l1_q16(a, b, len) -> (int64)(int32)sum |a - b|:
 * runtime-support/mind_intrinsics.c:1551-1562 (scalar), :1598-1608 (export). */
int64_t __mind_blas_dot_l1_q16(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_l1_q16_v (vector-dialect twin):
 * src/type_checker/mod.rs:2260, src/mlir/lowering.rs:2808-2817, :6035-6060. */
int64_t __mind_blas_dot_l1_q16_v(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_i16_v(a, b, len) -> (int64)(int32)sum a*b, int16
 * inputs: src/type_checker/mod.rs:2246, src/mlir/lowering.rs:5861-6030. */
int64_t __mind_blas_dot_i16_v(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_f32(a, b, len): strict-FP f32 dot (8 lanes of
 * unfused multiply-then-add, left-to-right lane fold, sequential tail); the
 * result's f32 bits are returned in the low 32 bits of the int64 (0 for
 * len <= 0 or NULL): runtime-support/mind_intrinsics.c:1190-1290.
 * The packed return has no room for an error code: a device failure also
 * returns 0 (the bits of +0.0f).  These symbols (and dotf32) clear
 * det_last_error() on entry, so a caller that must tell a failure from a
 * zero dot checks that det_last_error()[0] == '\0' after the call. */
int64_t __mind_blas_dot_f32(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_f32_v (vector-dialect twin, same schedule):
 * src/type_checker/mod.rs (dot_f32_v), src/mlir/lowering.rs:5528-5690. */
int64_t __mind_blas_dot_f32_v(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_l1_f32(a, b, len): sum of |a[i] - b[i]| (sign
 * bit cleared) on the dot's 8-lane schedule and fold; packed f32 bits, 0 for
 * len <= 0 or NULL (runtime-support/mind_intrinsics.c:1286-1351; arity
 * src/type_checker/mod.rs:2247).  Clears det_last_error() like the dot. */
int64_t __mind_blas_dot_l1_f32(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_l1_f32_v (vector-dialect twin, same schedule):
 * src/mlir/lowering.rs:6219-6401 (emit_vec_dot_metric_f32, L1). */
int64_t __mind_blas_dot_l1_f32_v(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_linf_f32(a, b, len): the largest |a[i] - b[i]|
 * from 0.0f, a NaN difference skipped as by the reference's scalar path and
 * its `d > m` test (runtime-support/mind_intrinsics.c:1355-1365; arity
 * type_checker:2258).  The reference's AVX2 path (:1367-1394, chosen at load
 * time on x86 hosts with AVX2) differs on NaN only: it returns NaN when a NaN
 * difference is the last one its lane 7 sees in the full 8-blocks (vmaxps
 * keeps its second operand). */
int64_t __mind_blas_dot_linf_f32(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_dot_linf_f32_v (arith.maximumf, lowering.rs:
 * 6219-6401): the same maximum, or a NaN (0x7fc00000) once any difference is
 * NaN. */
int64_t __mind_blas_dot_linf_f32_v(int64_t a, int64_t b, int64_t len);
/* Replaces __mind_blas_matmul_rmajor_f32(w, x, y, rows, cols): y[r] = the
 * strict dot of row r with x; -1 on a NULL pointer, 0 (y untouched) when
 * rows <= 0 or cols <= 0: runtime-support/mind_intrinsics.c:1418-1444. */
int64_t __mind_blas_matmul_rmajor_f32(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);
/* Replaces __mind_blas_matmul_rmajor_f32_v (vector-dialect twin):
 * src/mlir/lowering.rs:6441 (emit_vec_matmul_rmajor_f32).  Same values; a
 * NULL pointer returns 0 without writing (the emitted kernel has no check). */
int64_t __mind_blas_matmul_rmajor_f32_v(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);

/* ------------------------------------------------------------------------
 * Layer 2: the harness wrappers the reference benches and golden gate
 * dlsym (tests/cross_substrate_identity.rs:70-150, xnode_driver.c:123-125).
 * ---------------------------------------------------------------------- */
/* gemmi8: benches/det_matmul_i8.rs:120-129 */
int64_t gemmi8(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* gemmi8mt: tests/cross_substrate_identity.rs:106-108 */
int64_t gemmi8mt(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* gemmqmm (fused Q16, B is K x N): tests/cross_substrate_identity.rs:142-150 */
int64_t gemmqmm(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);
/* gemmq: Q16 GEMM with B given TRANSPOSED as bt[N][K] (the gemv-composed
 * form): tests/cross_substrate_identity.rs:82-94 */
int64_t gemmq(int64_t a, int64_t bt, int64_t c, int64_t m, int64_t k, int64_t n);
/* mmq / mmi16: tests/cross_substrate_identity.rs:76-81 */
int64_t mmq(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);
int64_t mmi16(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);
/* gemvq: benches/det_gemv_q16_mt.rs:90-94 */
int64_t gemvq(int64_t catalog, int64_t query, int64_t scores, int64_t m, int64_t k);
/* dotq: tests/cross_substrate_identity.rs:70-72 */
int64_t dotq(int64_t a, int64_t b, int64_t n);
/* dotl1q: tests/cross_substrate_identity/xnode_driver.c:149, :187 */
int64_t dotl1q(int64_t a, int64_t b, int64_t n);
/* doti16: tests/cross_substrate_identity/dot-i16-4096/manifest.toml (symbol) */
int64_t doti16(int64_t a, int64_t b, int64_t n);
/* dotf32 / mmf32: tests/cross_substrate_identity/{dot-f32-v-4093,
 * matmul-f32-v-64x64}/manifest.toml (symbol), cross_substrate_identity.rs:2579-2598 */
int64_t dotf32(int64_t a, int64_t b, int64_t n);
int64_t mmf32(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols);
/* fft256: the Q16.16 radix-2 DIT FFT symbol of examples/fft_q16.mind:15
 * (dlsym'd by benches/fft_q16.rs:255 and bench/fft/harness.c:62): re / im
 * are n int64 Q16.16 samples, transformed in place; tw holds n / 2 (wr, wi)
 * int64 pairs; n must be 2^logn (0 <= logn <= 30).  Returns 0; n == 0 does
 * nothing; any other (logn, n) returns DET_ERR_ARG (the reference indexes
 * out of its buffers there). */
int64_t fft256(int64_t re, int64_t im, int64_t tw, int64_t logn, int64_t n);

/* ------------------------------------------------------------------------
 * Layer 3: typed entry points of this build.
 * ---------------------------------------------------------------------- */
/* Host-pointer, synchronous.  Same contract as layer 1.  det_matmul_i16 is
 * the int16 GEMM whose every element is the reference int16 dot
 * (benches/det_matmul_i16.rs:218-224); the reference only has the GEMV. */
int64_t det_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k, int64_t n);
int64_t det_matmul_i16(const int16_t *a, const int16_t *b, int32_t *c, int64_t m, int64_t k, int64_t n);
int64_t det_matmul_q16(const int32_t *a, const int32_t *b, int32_t *c, int64_t m, int64_t k, int64_t n);
int64_t det_gemv_q16(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k);
/* nb independent queries: x is [nb][k], y is [nb][m]; equals nb calls of
 * __mind_blas_gemv_q16_mt (the reference takes one query per call). */
int64_t det_gemv_q16_batched(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k, int64_t nb);
int64_t det_gemv_i16(const int16_t *w, const int16_t *x, int32_t *y, int64_t m, int64_t k);
/* Vector reductions, returning (int64)(int32)sum like the reference:
 * Q16 dot (sum of per-term floors), Q16 L1 distance, int16 dot. */
int64_t det_dot_q16(const int32_t *a, const int32_t *b, int64_t len);
int64_t det_dot_l1_q16(const int32_t *a, const int32_t *b, int64_t len);
int64_t det_dot_i16(const int16_t *a, const int16_t *b, int64_t len);
/* Strict-FP f32 (same schedule as __mind_blas_dot_f32): *out receives the
 * dot; y[r] receives row r's dot with x.  Return 0 or a negative error. */
int64_t det_dot_f32(const float *a, const float *b, int64_t len, float *out);
int64_t det_matmul_rmajor_f32(const float *w, const float *x, float *y, int64_t rows, int64_t cols);
/* y[r] = metric op (DET_F32_*) of W row r and x, each exactly the value of
 * the matching single-vector symbol (dot / l1 / linf / linf_v) on that row:
 * one query against many rows (no reference counterpart; the batched form of
 * __mind_blas_dot_l1_f32 etc., as __mind_blas_matmul_rmajor_f32 is of the
 * dot).  cols == 0 gives +0.0f rows. */
int64_t det_rows_metric_f32(int64_t op, const float *w, const float *x, float *y, int64_t rows, int64_t cols);
/* batch independent fft256 transforms, transform f at re + f * n and
 * im + f * n (the reference transforms one per call); batch * n <= 2^31
 * points, else DET_ERR_ARG. */
int64_t det_fft_q16(int64_t *re, int64_t *im, const int64_t *tw, int64_t logn, int64_t n, int64_t batch);

/* Device-pointer, asynchronous on `stream` (a hipStream_t; NULL = default
 * stream).  Inputs must stay valid until the stream reaches the call.  The
 * i16 / q16 forms use a per-device workspace arena owned by the library
 * (grown with hipMalloc on demand; calls are ordered on it with an event);
 * det_matmul_ws_dev takes the workspace from the caller instead. */
int64_t det_matmul_i8_dev(const int8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                          void *stream);
int64_t det_matmul_i16_dev(const int16_t *a, const int16_t *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                           void *stream);
int64_t det_matmul_q16_dev(const int32_t *a, const int32_t *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                           void *stream);
int64_t det_gemv_q16_dev(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k, int64_t nb,
                         void *stream);
/* The batched Q16 GEMV (device form of __mind_blas_gemv_q16_mt,
 * src/mlir/lowering.rs:9822-9997, one call for nb query vectors) with the
 * workspace from the caller, like det_matmul_ws_dev: no arena, no
 * allocation, no event ordering between calls (calls sharing one workspace
 * must be ordered by the caller, e.g. on one stream).  The workspace holds
 * the query vectors' MFMA operands, det_gemv_workspace_bytes(m, k, nb) bytes
 * for 16-byte aligned w and 4-byte aligned x (0 when no group of vectors
 * takes the MFMA kernel); it is optional: with less, every vector runs the
 * one-vector kernel.  Its contents need not be initialised. */
int64_t det_gemv_workspace_bytes(int64_t m, int64_t k, int64_t nb);
int64_t det_gemv_q16_ws_dev(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k, int64_t nb,
                            void *ws, int64_t ws_bytes, void *stream);
int64_t det_gemv_i16_dev(const int16_t *w, const int16_t *x, int32_t *y, int64_t m, int64_t k, void *stream);
/* op = DET_DOT_Q16, DET_DOT_L1_Q16 or DET_DOT_I16; *out (device memory)
 * receives the int32 result (the reference's return value narrowed). */
int64_t det_dot_dev(int64_t op, const void *a, const void *b, int64_t len, int32_t *out, void *stream);
int64_t det_matmul_rmajor_f32_dev(const float *w, const float *x, float *y, int64_t rows, int64_t cols,
                                  void *stream);
int64_t det_rows_metric_f32_dev(int64_t op, const float *w, const float *x, float *y, int64_t rows, int64_t cols,
                                void *stream);
/* Device form of det_fft_q16 (n >= 4096 borrows the workspace arena, whose
 * size det_fft_workspace_bytes reports). */
int64_t det_fft_q16_dev(int64_t *re, int64_t *im, const int64_t *tw, int64_t logn, int64_t n, int64_t batch,
                        void *stream);
/* Out-of-place form: reads in_re / in_im, writes out_re / out_im (each pair
 * either identical, which is in place, or not overlapping). */
int64_t det_fft_q16_oop_dev(const int64_t *in_re, const int64_t *in_im, int64_t *out_re, int64_t *out_im,
                            const int64_t *tw, int64_t logn, int64_t n, int64_t batch, void *stream);
int64_t det_fft_workspace_bytes(int64_t logn, int64_t batch);
/* Workspace bytes op (DET_OP_*) needs at this shape (0 = none).
 *  - Tiny shapes run direct kernels that need none: int8 when its 16 x 16
 *    output tiles fit one round of the compute units and K <= 512, or
 *    K <= 4096 unless M, N and K are all multiples of 128 (every cube up to
 *    256^3, at any alignment); int16 under the same tile bound with
 *    K <= 4096; Q16 when those tiles fill at most 4 rounds and rounds times
 *    K is at most 4096 (every cube up to 512^3).
 *  - Otherwise int8 needs one only when K or N is not a multiple of 16: its
 *    operands are then repacked into aligned zero-padded panels of
 *    Mp*Kp + Kp*Np bytes (M, K, N rounded up to 256).  int8 operands that
 *    are not 16-byte aligned are repacked the same way when the workspace
 *    given holds that size, and so are aligned shapes of at least 256 rows
 *    and columns that no 128-row kernel takes, whose 256 x 256 tiles would
 *    not fill one round of the GPU and whose padding to multiples of 256 adds
 *    at most 1/8 per dimension (e.g. 1008^3), where the padded panels run
 *    faster.  For int8 the workspace is optional: without it such operands
 *    run a slower byte-load kernel; det_matmul_ws_dev rejects a short
 *    workspace only for int16 / Q16.
 *  - The figure holds for the current device: the rules above and the K
 *    split of mid-size Q16 grids (which keeps its partial sums in the
 *    workspace) depend on the device's compute-unit count, so ask on the
 *    device that runs the call. */
int64_t det_workspace_bytes(int64_t op, int64_t m, int64_t k, int64_t n);
int64_t det_matmul_ws_dev(int64_t op, const void *a, const void *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                          void *ws, int64_t ws_bytes, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): det_matmul_ws_dev with the workspace taken from a fixed
 * per-device array of DET_SCRATCH_BYTES compiled into the library, so the
 * call allocates nothing and never synchronises.  An int16 or Q16 shape
 * whose det_workspace_bytes exceeds it returns DET_ERR_ARG (32 MiB covers Q16
 * up to 1024^3 and int16 up to 2048^3); an int8 shape whose padded panels
 * exceed it runs the kernels that need no workspace instead.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, two host threads) race; order them. */
#define DET_SCRATCH_BYTES (32LL << 20)
int64_t det_matmul_scratch_dev(int64_t op, const void *a, const void *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                               void *stream);

/* Runtime helpers (thin wrappers over HIP, so a caller needs no HIP headers). */
/* Release the library's per-device state (its stream, events, host-call
 * staging buffers: device, pinned and the pinned ring, and workspace arena)
 * after waiting for the work queued on them, and join the host-copy
 * threads; later calls recreate what they need.  The reference joins its thread
 * pool at unload (runtime-support/mind_intrinsics.c:2066-2080); here the
 * release is explicit: a caller that unloads the library calls det_shutdown()
 * before dlclose (an exit hook would run HIP calls during process exit, which
 * abort under tools that intercept HIP).  No other call of the library may be
 * in flight. */
int64_t det_shutdown(void);
const char *det_last_error(void);
const char *det_version(void);
int64_t det_device_count(void);
int64_t det_set_device(int64_t d);
/* info[6]: CUs, max engine clock kHz, global memory bytes, LDS bytes per
 * workgroup, memory clock kHz, memory bus width bits. */
int64_t det_device_info(int64_t *info, char *name, int64_t name_len);
int64_t det_malloc(void **p, int64_t bytes);
int64_t det_free(void *p);
/* Synchronous: each returns once its bytes have landed, so work queued
 * afterwards on any stream (the library's streams do not wait for the null
 * stream) sees them. */
int64_t det_memcpy_htod(void *dst, const void *src, int64_t bytes);
int64_t det_memcpy_dtoh(void *dst, const void *src, int64_t bytes);
int64_t det_memset_dev(void *dst, int64_t byte, int64_t bytes);
int64_t det_device_sync(void);
int64_t det_stream_create(void **s);
int64_t det_stream_destroy(void *s);
int64_t det_stream_sync(void *s);
int64_t det_event_create(void **e);
int64_t det_event_destroy(void *e);
int64_t det_event_record(void *e, void *s);
int64_t det_event_elapsed_ms(void *start, void *stop, float *ms);

/* Roofline probes (no reference counterpart: they measure this GPU).
 * det_probe_mfma_i8: `blocks` x 256 threads issue 8 independent int8 MFMAs
 * per iteration on register operands (in: 128 x 16 bytes, out: blocks*256
 * ints); shape 0 = 16x16x64, 1 = 32x32x32;
 * ops = blocks * 4 * iters * 8 * (16384 or 32768) * 2; shape 2 = 32x32x32
 * cycling 8 operand pairs, 16 MFMAs per iteration (in: 1024 x 16 bytes),
 * ops = blocks * 4 * iters * 16 * 32768 * 2; shape 3 = 16x16x64 cycling
 * 8 operand pairs, 32 MFMAs per iteration (in: 1024 x 16 bytes),
 * ops = blocks * 4 * iters * 32 * 16384 * 2.  det_probe_read streams
 * `bytes` once (out: `blocks` zeroed words).  det_copy_dev is the plain copy
 * kernel of known size that calibrates the profiler's byte counters. */
int64_t det_probe_mfma_i8(const void *in, int32_t *out, int64_t blocks, int64_t iters, int64_t shape,
                          void *stream);
int64_t det_probe_read(const void *src, int64_t bytes, uint32_t *out, int64_t blocks, void *stream);
int64_t det_copy_dev(void *dst, const void *src, int64_t bytes, void *stream);

/* Seeded input generators of the reference bench harness (LCG
 * benches/det_matmul_q16.rs:196-209; draw A then B). */
void det_gen_i8(uint64_t seed, int8_t *a, int64_t na, int8_t *b, int64_t nb);
void det_gen_i16(uint64_t seed, int16_t *a, int64_t na, int16_t *b, int64_t nb);
void det_gen_q16(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb);
void det_gen_q16_sat(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb);
void det_gen_i8_gauss(uint64_t seed, int8_t *x, int64_t n);
void det_gen_i8_sym127(uint64_t seed, int8_t *w, int64_t n);
/* f32 samples ((float)u32 / (float)UINT32_MAX) * 2 - 1, A then B
 * (tests/cross_substrate_identity.rs make_pair_f32). */
void det_gen_f32_unit(uint64_t seed, float *a, int64_t na, float *b, int64_t nb);

#ifdef __cplusplus
}
#endif
#endif /* MIND_DET_H */
