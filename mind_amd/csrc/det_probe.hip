// det_probe.hip -- micro-kernels that measure this GPU's roofline denominators
// (int8 MFMA issue rate, HBM read and copy bandwidth) and a plain copy kernel
// of known size used to calibrate the profiler's HBM byte counters.
#include "det_common.h"
#include "../../include/mind_det.h"

namespace det {
namespace probe {

// Every wave issues `iters` rounds of 8 independent int8 MFMAs on register
// operands (no memory traffic).  The MFMAs are emitted as inline assembly so
// the loop holds nothing else: the compiler's register allocation cannot add
// accumulator moves, and each accumulator chain has 7 other MFMAs between its
// dependent issues.  SHAPE 0: 16x16x64 (16384 MACs), SHAPE 1: 32x32x32
// (32768 MACs), both with one operand pair for all MFMAs.  SHAPE 2:
// 32x32x32 with 8 different operand pairs (A from in[64 c + l], B from
// in[512 + 64 c + l]), cycled so consecutive MFMAs see different data: with
// random operands this is the issue rate a GEMM's data allows, since the
// clock under int8 MFMA load depends on how many operand bits toggle.
// SHAPE 3: the same for 16x16x64 (32 MFMAs per round, the MACs of 16
// 32x32x32), the instruction the int8 GEMM kernels issue.
template <int SHAPE>
__global__ __launch_bounds__(256) void mfma_i8_kernel(const v2i64 *__restrict__ in, int *__restrict__ out, int iters) {
    const int l = threadIdx.x & 63;
    const v2i64 a = in[l], b = in[64 + l];
    int s = 0;
    if (SHAPE == 3) {
        v2i64 x[8], y[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            x[c] = in[64 * c + l];
            y[c] = in[512 + 64 * c + l];
        }
        v4i32 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
        for (int it = 0; it < iters; ++it) {
#define MF(c, i, j) asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(c) : "v"(x[i]), "v"(y[j]))
            MF(c0, 0, 0); MF(c1, 1, 1); MF(c2, 2, 2); MF(c3, 3, 3); MF(c4, 4, 4); MF(c5, 5, 5); MF(c6, 6, 6); MF(c7, 7, 7);
            MF(c0, 1, 2); MF(c1, 2, 3); MF(c2, 3, 4); MF(c3, 4, 5); MF(c4, 5, 6); MF(c5, 6, 7); MF(c6, 7, 0); MF(c7, 0, 1);
            MF(c0, 2, 4); MF(c1, 3, 5); MF(c2, 4, 6); MF(c3, 5, 7); MF(c4, 6, 0); MF(c5, 7, 1); MF(c6, 0, 2); MF(c7, 1, 3);
            MF(c0, 3, 6); MF(c1, 4, 7); MF(c2, 5, 0); MF(c3, 6, 1); MF(c4, 7, 2); MF(c5, 0, 3); MF(c6, 1, 4); MF(c7, 2, 5);
#undef MF
        }
        asm volatile("s_nop 7\n s_nop 7" ::);
        const v4i32 t = c0 ^ c1 ^ c2 ^ c3 ^ c4 ^ c5 ^ c6 ^ c7;
        s = t.x ^ t.y ^ t.z ^ t.w;
    } else if (SHAPE == 2) {
        v2i64 x[8], y[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            x[c] = in[64 * c + l];
            y[c] = in[512 + 64 * c + l];
        }
        v16i32 c0 = {0}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
        for (int it = 0; it < iters; ++it) {
#define MF(c, i, j) asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(c) : "v"(x[i]), "v"(y[j]))
            MF(c0, 0, 0); MF(c1, 1, 1); MF(c2, 2, 2); MF(c3, 3, 3); MF(c4, 4, 4); MF(c5, 5, 5); MF(c6, 6, 6); MF(c7, 7, 7);
            MF(c0, 1, 2); MF(c1, 2, 3); MF(c2, 3, 4); MF(c3, 4, 5); MF(c4, 5, 6); MF(c5, 6, 7); MF(c6, 7, 0); MF(c7, 0, 1);
#undef MF
        }
        asm volatile("s_nop 7\n s_nop 7\n s_nop 7" ::);
        const v16i32 t = c0 ^ c1 ^ c2 ^ c3 ^ c4 ^ c5 ^ c6 ^ c7;
        for (int i = 0; i < 16; ++i) s ^= t[i];
    } else if (SHAPE == 0) {
        v4i32 c0 = {0, 0, 0, 1}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
        for (int it = 0; it < iters; ++it) {
#define MF(c) asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b))
            MF(c0); MF(c1); MF(c2); MF(c3); MF(c4); MF(c5); MF(c6); MF(c7);
#undef MF
        }
        asm volatile("s_nop 7\n s_nop 7" ::);
        const v4i32 t = c0 ^ c1 ^ c2 ^ c3 ^ c4 ^ c5 ^ c6 ^ c7;
        s = t.x ^ t.y ^ t.z ^ t.w;
    } else {
        v16i32 c0 = {0}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
        for (int it = 0; it < iters; ++it) {
#define MF(c) asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b))
            MF(c0); MF(c1); MF(c2); MF(c3); MF(c4); MF(c5); MF(c6); MF(c7);
#undef MF
        }
        asm volatile("s_nop 7\n s_nop 7\n s_nop 7" ::);
        const v16i32 t = c0 ^ c1 ^ c2 ^ c3 ^ c4 ^ c5 ^ c6 ^ c7;
        for (int i = 0; i < 16; ++i) s ^= t[i];
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Streaming read: XOR of all 16-byte words, one result per workgroup.
__global__ __launch_bounds__(256) void read_kernel(const uint4 *__restrict__ src, size_t n16, uint32_t *__restrict__ out) {
    uint32_t x = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
        const v4i32 v = __builtin_nontemporal_load((const v4i32 *)src + i);
        x ^= (uint32_t)(v.x ^ v.y ^ v.z ^ v.w);
    }
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if ((threadIdx.x & 63) == 0) atomicXor(out + blockIdx.x, x);
}

__global__ __launch_bounds__(256) void copy_kernel(uint4 *__restrict__ dst, const uint4 *__restrict__ src, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

}  // namespace probe
}  // namespace det

extern "C" {

// in: 128 x 16 bytes of operands (shapes 0, 1) or 1024 x 16 (shapes 2, 3),
// out: blocks*256 ints.  Returns the launch status; ops per launch = blocks *
// 4 waves * iters * MFMAs * MACs * 2: 8 x 16384 (shape 0, 16x16x64),
// 8 x 32768 (shape 1, 32x32x32), 16 x 32768 (shape 2, 32x32x32 cycling
// 8 operand pairs), 32 x 16384 (shape 3, 16x16x64 cycling 8 operand pairs).
int64_t det_probe_mfma_i8(const void *in, int32_t *out, int64_t blocks, int64_t iters, int64_t shape, void *stream) {
    if (!in || !out || blocks <= 0 || iters <= 0 || blocks > (1 << 20) || iters > (1 << 30) || shape < 0 || shape > 3)
        return det_fail(DET_ERR_ARG, "bad det_probe_mfma_i8 arguments");
    if (shape == 0)
        hipLaunchKernelGGL(det::probe::mfma_i8_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const det::v2i64 *)in, out, (int)iters);
    else if (shape == 1)
        hipLaunchKernelGGL(det::probe::mfma_i8_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const det::v2i64 *)in, out, (int)iters);
    else if (shape == 3)
        hipLaunchKernelGGL(det::probe::mfma_i8_kernel<3>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const det::v2i64 *)in, out, (int)iters);
    else
        hipLaunchKernelGGL(det::probe::mfma_i8_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const det::v2i64 *)in, out, (int)iters);
    DET_HIP_CHECK(hipGetLastError());
    return 0;
}

// Streams `bytes` (multiple of 16) once; out needs `blocks` uint32 (zeroed).
int64_t det_probe_read(const void *src, int64_t bytes, uint32_t *out, int64_t blocks, void *stream) {
    if (!src || !out || bytes <= 0 || (bytes & 15) || blocks <= 0 || blocks > (1 << 20))
        return det_fail(DET_ERR_ARG, "bad det_probe_read arguments");
    hipLaunchKernelGGL(det::probe::read_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)src, (size_t)bytes / 16, out);
    DET_HIP_CHECK(hipGetLastError());
    return 0;
}

// dst <- src, `bytes` a multiple of 16: the plain copy kernel of known size.
int64_t det_copy_dev(void *dst, const void *src, int64_t bytes, void *stream) {
    if (!dst || !src || bytes < 0 || (bytes & 15)) return det_fail(DET_ERR_ARG, "bad det_copy_dev arguments");
    if (bytes == 0) return 0;
    const size_t n16 = (size_t)bytes / 16;
    const unsigned blocks = (unsigned)(n16 / 256 < 8192 ? (n16 + 255) / 256 : 8192);
    hipLaunchKernelGGL(det::probe::copy_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (uint4 *)dst,
                       (const uint4 *)src, n16);
    DET_HIP_CHECK(hipGetLastError());
    return 0;
}

}  // extern "C"
