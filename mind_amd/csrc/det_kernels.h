// det_kernels.h -- kernel launchers shared between the kernel files and the
// C-ABI layer.  All pointers are device pointers; every launcher is
// asynchronous on `s` and returns the launch status.  Shapes must already be
// validated (0 < M, N; 0 <= K; all below 2^31).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace det {

// Compute units of the current device (cached per device; 256 if unknown).
int cu_count();

// The int16 and Q16 preps write column sums of B as at most MAX_CS exact
// partials per column ([ncs][N], ncs <= MAX_CS); the GEMM epilogues add them.
constexpr int MAX_CS = 16;

// C[M,N] (i32) = A[M,K] (i8) * B[K,N] (i8).  Shapes off the 16-byte grid (K
// or N not a multiple of 16, operands not 16-byte aligned), and the small
// on-grid shapes the edge kernel would underfill (i8_edge_underfills),
// repack the operands into `ws`, which must then hold i8_workspace_bytes(M,
// N, K, aligned) bytes (0 for every other shape; with ws == NULL they take
// the byte-load or edge kernel instead).
size_t i8_workspace_bytes(int M, int N, int K, bool aligned);
// Tiny int8 shapes (det_gemm_small.hip): one direct v_dot4 launch, no
// workspace, any alignment, when the 16x16 output tiles fit one round of the
// compute units and K <= I8_SMALL_K, or K <= I8_SMALL_K_ODD for shapes the
// full-tile MFMA kernels do not take (M, N or K not a multiple of 128).
constexpr long long I8_SMALL_K = 512, I8_SMALL_K_ODD = 4096;
bool i8_small(int M, int N, int K);
hipError_t launch_gemm_i8_small(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, hipStream_t s);
// The same for int16 (v_dot2 kernel), K <= I16_SMALL_K.
constexpr long long I16_SMALL_K = 4096;
bool i16_small(int M, int N, int K);
hipError_t launch_gemm_i16_small(const int16_t *A, const int16_t *B, int32_t *C, int M, int N, int K,
                                 hipStream_t s);
hipError_t launch_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, void *ws,
                          hipStream_t s);

// Workspace (device bytes) the limb GEMMs need: operand limb planes, low-16
// halves (Q16) and exact row / column sums.
size_t limb_workspace_bytes(int M, int N, int K, int np, bool q16);
size_t q16x_workspace_bytes(int M, int N, int K);   // the second-generation Q16 kernel's layout
// Small Q16 shapes (det_gemm_q16s.hip): one direct launch, no workspace,
// when the 16x16 output tiles fill at most Q16_SMALL_ROUNDS rounds of the
// compute units and rounds times K is at most Q16_SMALL_TERMS.
constexpr long long Q16_SMALL_ROUNDS = 4, Q16_SMALL_TERMS = 4096;
bool q16_small(int M, int N, int K);
hipError_t launch_gemm_q16_small(const int32_t *A, const int32_t *B, int32_t *C, int M, int N, int K, bool b_is_t,
                                 hipStream_t s);
inline size_t q16_workspace_bytes(int M, int N, int K) {
    if (q16_small(M, N, K)) return 0;
    const size_t a = limb_workspace_bytes(M, N, K, 4, true), b = q16x_workspace_bytes(M, N, K);
    return a > b ? a : b;
}
size_t i16_workspace_bytes(int M, int N, int K);   // covers both int16 paths below

// Q16.16: B is [K][N], or [N][K] when b_is_t.
hipError_t launch_gemm_q16(const int32_t *A, const int32_t *B, int32_t *C, int M, int N, int K, bool b_is_t,
                           void *ws, hipStream_t s);
// Second-generation Q16 kernel (12 waves per 64x64 tile, no flush): eligible
// for 1 <= K < 65536 (the shift-0/1 limb sets stay exact in int32 only below
// 2^16 terms) and 6 * (M + N) * Kp < 2^31 (Kp = K rounded up to 64).  Its
// workspace is covered by q16_workspace_bytes.
bool q16x_eligible(int M, int N, int K);
hipError_t launch_gemm_q16x(const int32_t *A, const int32_t *B, int32_t *C, int M, int N, int K, bool b_is_t,
                            void *ws, hipStream_t s);
hipError_t launch_gemm_i16(const int16_t *A, const int16_t *B, int32_t *C, int M, int N, int K, void *ws,
                           hipStream_t s);
// int16 as one int8 MFMA GEMM on interleaved limbs (det_gemm_i16x.hip):
// eligible when 2*M*Kp and Kp*round_up(2N, 16) are below 2^31 (Kp = K
// rounded up to 16).
bool i16x_eligible(int M, int N, int K);
size_t i16x_workspace_bytes(int M, int N, int K);
hipError_t launch_gemm_i16x(const int16_t *A, const int16_t *B, int32_t *C, int M, int N, int K, void *ws,
                            hipStream_t s);

// Y[nb][M] = Q16 GEMV of W[M][K] with each X[b][K].
hipError_t launch_gemv_q16(const int32_t *W, const int32_t *X, int32_t *Y, int M, int K, int nb, hipStream_t s);
// Several query vectors at once (nb <= 8) on the int8 MFMA + VALU residue:
// eligible when M >= 16, K % 512 == 0, K <= 32768, W < 2^31 bytes, aligned.
bool gemv8_eligible(const int32_t *W, const int32_t *X, int M, int K);
size_t gemv8_workspace_bytes(int K);
hipError_t launch_gemv_q16_mfma(const int32_t *W, const int32_t *X, int32_t *Y, int M, int K, int nb, void *ws,
                                hipStream_t s);
// Vector reductions: sum mod 2^32 of the Q16 per-term floor products
// (DOT_Q16), of |a - b| (DOT_L1, int32 inputs) or of int16 products
// (DOT_I16); *out (one device uint32) is overwritten.
enum { DOT_Q16 = 0, DOT_L1 = 1, DOT_I16 = 2 };
hipError_t launch_dot(int op, const void *a, const void *b, int64_t n, uint32_t *out, hipStream_t s);
// True when one block covers the dot (n <= 16384): it then stores its sum
// (no atomic, no zeroing launch), so *out may be host memory.
bool dot_single_block(int64_t n);
// Strict-FP f32: y[r] = metric met of W row r and x on the reference's
// pinned 8-lane schedule: F32_DOT (no fused multiply-add, fixed fold order),
// F32_L1 (sum of sign-cleared differences), F32_LINF (max, NaN skipped),
// F32_LINF_V (max, NaN once any difference is NaN); rows > 0, cols > 0.
enum { F32_DOT = 0, F32_L1 = 1, F32_LINF = 2, F32_LINF_V = 3 };
hipError_t launch_rows_f32(const float *W, const float *x, float *y, int64_t rows, int64_t cols, int met,
                           hipStream_t s);
// y[M] = int16 GEMV.
hipError_t launch_gemv_i16(const int16_t *W, const int16_t *x, int32_t *y, int M, int K, hipStream_t s);

// Q16.16 radix-2 DIT FFT (det_fft.hip): batch transforms of 2^logn points
// from (sre, sim) to (dre, dim) (the same pointers for in place); ws holds
// fft_workspace_bytes(logn, batch) bytes (0 for logn <= 11).
size_t fft_workspace_bytes(int logn, int64_t batch);
hipError_t launch_fft_q16(const int64_t *sre, const int64_t *sim, int64_t *dre, int64_t *dim, const int64_t *tw,
                          int logn, int64_t batch, void *ws, hipStream_t s);

}  // namespace det
