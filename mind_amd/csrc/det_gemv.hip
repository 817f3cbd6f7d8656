// det_gemv.hip -- exact Q16.16 and int16 GEMV, HBM-streaming.
//
//   y[b][i] = (int32) sum_k ( (int64)W[i,k] * (int64)x[b][k]  >>arith 16 )
// Semantics of __mind_blas_gemv_q16_mt / __mind_blas_matmul_rmajor_q16_v
// (reference src/mlir/lowering.rs:9822-9997 emit_gemv_q16_row_band and
// :6675-7035; oracle benches/det_gemv_q16_mt.rs:186-197 and the per-row
// runtime-support/mind_intrinsics.c:1459-1471 dot).
//
// Per term the kernel needs bits [16, 48) of the 64-bit product, i.e.
// alignbit(mul_hi_i32(w, x), mul_lo_u32(w, x), 16); summing those mod 2^32 is
// exactly the reference's i64 sum of floor-shifted terms truncated to i32
// (the truncation only keeps the low 32 bits, and each term's low 32 bits
// are the alignbit result).  Integer addition is associative, so the
// per-lane partial sums and the wave reduction give the same bits in any
// order.
//
// W is read exactly once with 16-byte loads: each wave owns ROWS rows and
// its 64 lanes sweep K in 16-byte columns, so one load instruction moves
// 1 KiB of one row; the x chunk loaded by a lane is reused for all ROWS rows
// (and x stays L2 resident: 64 KiB per vector).
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace gemv {

constexpr int THREADS = 256, WAVES = THREADS / 64;

__device__ __forceinline__ uint32_t q16_term(int32_t w, int32_t x) {
    const uint32_t lo = (uint32_t)w * (uint32_t)x;
    const uint32_t hi = (uint32_t)__mulhi(w, x);
    return __builtin_amdgcn_alignbit(hi, lo, 16);
}

// 16-byte streaming load of column c (non-temporal: W is read exactly once)
__device__ __forceinline__ int4 ntload4(const void *base, int c) {
    const v4i32 v = __builtin_nontemporal_load((const v4i32 *)base + c);
    return make_int4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// FAST: K % 4 == 0 and W, x 16-byte aligned.  NB: number of vectors.
template <int ROWS, int NB, bool FAST>
__global__ __launch_bounds__(THREADS) void gemv_q16_kernel(const int32_t *__restrict__ W,
                                                          const int32_t *__restrict__ X,
                                                          int32_t *__restrict__ Y, int M, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * ROWS;
    if (row0 >= M) return;
    uint32_t acc[NB][ROWS];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[b][r] = 0;

    const int32_t *wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) wr[r] = W + (size_t)min(row0 + r, M - 1) * K;

    if (FAST) {
        const int K4 = K >> 2;                  // 16-byte columns
        constexpr int U = 2;                    // columns per lane per trip
        int c = lane;
        for (; c + 64 * (U - 1) < K4; c += 64 * U) {
            int4 wv[U][ROWS];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) wv[u][r] = ntload4(wr[r], c + 64 * u);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const int4 xv = *((const int4 *)(X + (size_t)b * K) + c + 64 * u);
#pragma unroll
                    for (int r = 0; r < ROWS; ++r) {
                        acc[b][r] += q16_term(wv[u][r].x, xv.x);
                        acc[b][r] += q16_term(wv[u][r].y, xv.y);
                        acc[b][r] += q16_term(wv[u][r].z, xv.z);
                        acc[b][r] += q16_term(wv[u][r].w, xv.w);
                    }
                }
        }
        for (; c < K4; c += 64) {
            int4 wv[ROWS];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) wv[r] = ntload4(wr[r], c);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int4 xv = *((const int4 *)(X + (size_t)b * K) + c);
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    acc[b][r] += q16_term(wv[r].x, xv.x);
                    acc[b][r] += q16_term(wv[r].y, xv.y);
                    acc[b][r] += q16_term(wv[r].z, xv.z);
                    acc[b][r] += q16_term(wv[r].w, xv.w);
                }
            }
        }
    } else {
        for (int k = lane; k < K; k += 64) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int32_t xv = X[(size_t)b * K + k];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) acc[b][r] += q16_term(wr[r][k], xv);
            }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint32_t s = wave_sum(acc[b][r]);
            if (lane == 0 && row0 + r < M) Y[(size_t)b * M + row0 + r] = (int32_t)s;
        }
}

template <int ROWS, int NB>
static void launch_rows(const int32_t *W, const int32_t *X, int32_t *Y, int M, int K, bool fast, hipStream_t s) {
    const dim3 grid((M + WAVES * ROWS - 1) / (WAVES * ROWS)), block(THREADS);
    if (fast)
        hipLaunchKernelGGL((gemv_q16_kernel<ROWS, NB, true>), grid, block, 0, s, W, X, Y, M, K);
    else
        hipLaunchKernelGGL((gemv_q16_kernel<ROWS, NB, false>), grid, block, 0, s, W, X, Y, M, K);
}

}  // namespace gemv

// X: [nb][K], Y: [nb][M].  Batches are processed 8 (then 4, 2, 1) at a time
// so that W is streamed once per group of up to 8 vectors.
hipError_t launch_gemv_q16(const int32_t *W, const int32_t *X, int32_t *Y, int M, int K, int nb, hipStream_t s) {
    using namespace gemv;
    const bool fast = (K % 4 == 0) && (((uintptr_t)W & 15) == 0) && (((uintptr_t)X & 15) == 0);
    int b = 0;
    while (b < nb) {
        const int left = nb - b;
        const int32_t *Xb = X + (size_t)b * K;
        int32_t *Yb = Y + (size_t)b * M;
        if (left >= 8) { launch_rows<2, 8>(W, Xb, Yb, M, K, fast, s); b += 8; }
        else if (left >= 4) { launch_rows<2, 4>(W, Xb, Yb, M, K, fast, s); b += 4; }
        else if (left >= 2) { launch_rows<4, 2>(W, Xb, Yb, M, K, fast, s); b += 2; }
        else { launch_rows<4, 1>(W, Xb, Yb, M, K, fast, s); b += 1; }
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ int16
// y[r] = (int32) sum_i (int64)W[r,i] * (int64)x[i]
// (__mind_blas_matmul_rmajor_i16_v; reference src/mlir/lowering.rs:
// 10723-11150, oracle benches/det_matmul_i16.rs:218-230).  Only the low 32
// bits survive the final truncation, so the i32 products of the
// sign-extended halves (v_mul_i32_i24 is exact for 16-bit operands) summed
// mod 2^32 are the exact result.
namespace gemv {
template <int ROWS, bool FAST>
__global__ __launch_bounds__(THREADS) void gemv_i16_kernel(const int16_t *__restrict__ W,
                                                          const int16_t *__restrict__ x,
                                                          int32_t *__restrict__ y, int M, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * WAVES + wave) * ROWS;
    if (row0 >= M) return;
    uint32_t acc[ROWS];
    const int16_t *wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        acc[r] = 0;
        wr[r] = W + (size_t)min(row0 + r, M - 1) * K;
    }
    if (FAST) {
        const int K8 = K >> 3;   // 16-byte columns of 8 int16
        for (int c = lane; c < K8; c += 64) {
            const int4 xv = *((const int4 *)x + c);
            const int xs[8] = {(int16_t)xv.x, xv.x >> 16, (int16_t)xv.y, xv.y >> 16,
                               (int16_t)xv.z, xv.z >> 16, (int16_t)xv.w, xv.w >> 16};
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const int4 wv = ntload4(wr[r], c);
                const int ws[8] = {(int16_t)wv.x, wv.x >> 16, (int16_t)wv.y, wv.y >> 16,
                                   (int16_t)wv.z, wv.z >> 16, (int16_t)wv.w, wv.w >> 16};
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r] += (uint32_t)(ws[e] * xs[e]);
            }
        }
    } else {
        for (int k = lane; k < K; k += 64) {
            const int xv = x[k];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] += (uint32_t)((int)wr[r][k] * xv);
        }
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const uint32_t s = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < M) y[row0 + r] = (int32_t)s;
    }
}
}  // namespace gemv

hipError_t launch_gemv_i16(const int16_t *W, const int16_t *x, int32_t *y, int M, int K, hipStream_t s) {
    using namespace gemv;
    constexpr int ROWS = 4;
    const bool fast = (K % 8 == 0) && (((uintptr_t)W & 15) == 0) && (((uintptr_t)x & 15) == 0);
    const dim3 grid((M + WAVES * ROWS - 1) / (WAVES * ROWS)), block(THREADS);
    if (fast)
        hipLaunchKernelGGL((gemv_i16_kernel<ROWS, true>), grid, block, 0, s, W, x, y, M, K);
    else
        hipLaunchKernelGGL((gemv_i16_kernel<ROWS, false>), grid, block, 0, s, W, x, y, M, K);
    return hipGetLastError();
}

}  // namespace det
