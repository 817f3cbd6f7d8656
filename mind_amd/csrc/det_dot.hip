// det_dot.hip -- exact vector reductions: Q16.16 dot, Q16.16 L1 distance and
// int16 dot, each returned as (int64)(int32)sum like the reference.
//
//   DOT_Q16 : sum_k ((int64)a[k] * (int64)b[k]) >>arith 16
//             (__mind_blas_dot_q16 / _v: runtime-support/mind_intrinsics.c:
//             1459-1471, lowering.rs emit_vec_dot_q16 :5695-5860)
//   DOT_L1  : sum_k |(int64)a[k] - (int64)b[k]|
//             (__mind_blas_dot_l1_q16 / _v: mind_intrinsics.c:1551-1562,
//             lowering.rs emit_vec_dot_l1_q16 :6035-6060)
//   DOT_I16 : sum_k (int64)a[k] * (int64)b[k]   (int16 inputs)
//             (__mind_blas_dot_i16_v: lowering.rs emit_vec_dot_i16 :5861)
//
// The reference accumulates in int64 and keeps the low 32 bits, so every
// term only matters mod 2^32: the Q16 term is bits [16, 48) of the 64-bit
// product (v_alignbit of mul_hi / mul_lo), the L1 term |a - b| < 2^32 is the
// unsigned difference of the larger and the smaller value, and the int16
// product is exact in 32 bits.  Sums are uint32 with wrap-around.  Integer
// addition mod 2^32 is associative and commutative, so the grid-wide sum
// (one integer atomic per block) is the same number in any order.  A dot
// that one block covers stores its sum instead (no atomic, so no zeroing
// launch, and the output may be host memory).
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace dot {

constexpr int THREADS = 256;
constexpr int64_t PER_THREAD = 64;   // elements per thread at which another block is added

template <int OP>
__device__ __forceinline__ uint32_t term(uint32_t a, uint32_t b) {
    if (OP == DOT_Q16) {
        const uint32_t lo = a * b;
        const uint32_t hi = (uint32_t)__mulhi((int)a, (int)b);
        return __builtin_amdgcn_alignbit(hi, lo, 16);
    } else if (OP == DOT_L1) {
        const bool ge = (int32_t)a >= (int32_t)b;
        return ge ? a - b : b - a;
    } else {
        return (uint32_t)((int32_t)(int16_t)a * (int32_t)(int16_t)b);
    }
}

// Elements are read as 16-byte vectors where the whole vector is in range
// (aligned bases only) and one at a time in the tail.
template <int OP>
__global__ __launch_bounds__(THREADS) void dot_kernel(const void *__restrict__ A, const void *__restrict__ B, int64_t n,
                                                      uint32_t *__restrict__ out, bool vec) {
    constexpr int EB = OP == DOT_I16 ? 2 : 4;      // element bytes
    constexpr int PER = 16 / EB;                   // elements per 16-byte vector
    uint32_t acc = 0;
    const int64_t nvec = vec ? n / PER : 0;
    const int64_t stride = (int64_t)gridDim.x * THREADS;
    for (int64_t v = (int64_t)blockIdx.x * THREADS + threadIdx.x; v < nvec; v += stride) {
        const uint4 x = ((const uint4 *)A)[v], y = ((const uint4 *)B)[v];
        const uint32_t xa[4] = {x.x, x.y, x.z, x.w}, ya[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (EB == 4) {
                acc += term<OP>(xa[e], ya[e]);
            } else {
                acc += term<OP>(xa[e] & 0xffffu, ya[e] & 0xffffu);
                acc += term<OP>(xa[e] >> 16, ya[e] >> 16);
            }
        }
    }
    for (int64_t i = nvec * PER + (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += stride) {
        const uint32_t a = EB == 4 ? ((const uint32_t *)A)[i] : (uint32_t)((const uint16_t *)A)[i];
        const uint32_t b = EB == 4 ? ((const uint32_t *)B)[i] : (uint32_t)((const uint16_t *)B)[i];
        acc += term<OP>(a, b);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += (uint32_t)__shfl_xor((int)acc, off);
    __shared__ uint32_t part[THREADS / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < THREADS / 64; ++w) s += part[w];
        if (gridDim.x == 1) *out = s;
        else atomicAdd(out, s);
    }
}

__global__ void zero_u32(uint32_t *p) { *p = 0; }

}  // namespace dot

bool dot_single_block(int64_t n) { return n <= (int64_t)dot::THREADS * dot::PER_THREAD; }

// out: one uint32, overwritten with sum mod 2^32 (device memory; host memory
// too when dot_single_block(n)).
hipError_t launch_dot(int op, const void *a, const void *b, int64_t n, uint32_t *out, hipStream_t s) {
    using namespace dot;
    if (n <= 0 || !dot_single_block(n)) hipLaunchKernelGGL(zero_u32, dim3(1), dim3(1), 0, s, out);
    if (n <= 0) return hipGetLastError();
    const bool vec = (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
    const int64_t blocks = (n + THREADS * PER_THREAD - 1) / (THREADS * PER_THREAD);
    const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024));
    switch (op) {
    case DOT_Q16: hipLaunchKernelGGL(dot_kernel<DOT_Q16>, grid, dim3(THREADS), 0, s, a, b, n, out, vec); break;
    case DOT_L1: hipLaunchKernelGGL(dot_kernel<DOT_L1>, grid, dim3(THREADS), 0, s, a, b, n, out, vec); break;
    case DOT_I16: hipLaunchKernelGGL(dot_kernel<DOT_I16>, grid, dim3(THREADS), 0, s, a, b, n, out, vec); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace det
