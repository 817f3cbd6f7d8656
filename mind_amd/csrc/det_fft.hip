// det_fft.hip -- deterministic Q16.16 radix-2 DIT FFT, batched, in place.
//
// Semantics (examples/fft_q16.mind:15-120, the fft256(re, im, tw, logn, n)
// symbol that benches/fft_q16.rs:66-168 and bench/fft/harness.c dlopen):
// re / im are n = 2^logn int64 Q16.16 samples; tw[2k], tw[2k+1] (k < n/2) the
// twiddle (wr, wi).  After the bit-reversal permutation, the span-2 stage is
// a plain add / subtract (the kernel peels it: no twiddle), and every span
// s >= 4 stage runs, for each block base and j < s/2, with k = j * (n / s):
//     t = (qmul(wr, x_b) - qmul(wi, y_b),  qmul(wr, y_b) + qmul(wi, x_b))
//     a' = a + t,  b' = a - t,        qmul(w, v) = low64(w * v) >>arith 16
// All adds, subtracts and products wrap in int64, like MIND's i64 ops.
//
// GPU mapping.  Butterflies of one stage are independent, and the stage
// order is all that the result depends on, so any data layout that performs
// the same butterflies stage by stage gives the same bits.  The position
// (after bit reversal) of a point is a logn-bit number; stage b pairs points
// that differ in bit b.  A pass keeps 16 points per lane whose positions
// differ exactly in a 4-bit window [s, s + 4) (register index r = those
// bits, lane index t = the other bits) and runs the stages of that window in
// registers:
//   * n <= 16        : one FFT per thread (fft_small_kernel);
//   * 32 <= n <= 2048: n / 16 lanes per FFT, passes separated by an LDS
//                      transpose, bit reversal folded into the first load,
//                      one HBM read and one write per point (fft_lds_kernel);
//   * n >= 4096      : one global-memory pass per 4-bit window, out of place
//                      through a workspace (fft_pass_kernel).
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace fft {

__device__ __forceinline__ int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
__device__ __forceinline__ int64_t wsub(int64_t a, int64_t b) { return (int64_t)((uint64_t)a - (uint64_t)b); }
__device__ __forceinline__ int64_t qmul(int64_t w, int64_t v) {
    return ((int64_t)((uint64_t)w * (uint64_t)v)) >> 16;
}

// One butterfly of stage b (b == 0: the peeled span-2 stage) on (a, b).
__device__ __forceinline__ void butterfly(int64_t &ar, int64_t &ai, int64_t &br, int64_t &bi, int64_t wr, int64_t wi,
                                          bool peeled) {
    int64_t tr, ti;
    if (peeled) {
        tr = br, ti = bi;
    } else {
        tr = wsub(qmul(wr, br), qmul(wi, bi));
        ti = wadd(qmul(wr, bi), qmul(wi, br));
    }
    const int64_t ur = ar, ui = ai;
    ar = wadd(ur, tr), ai = wadd(ui, ti);
    br = wsub(ur, tr), bi = wsub(ui, ti);
}

__device__ __forceinline__ uint32_t bitrev(uint32_t v, int bits) { return bits ? __brev(v) >> (32 - bits) : 0u; }

// Position of register r of lane-group index t for the window [s, s + 4).
__device__ __forceinline__ uint32_t win_pos(uint32_t t, int r, int s) {
    return ((t >> s) << (s + 4)) | ((uint32_t)r << s) | (t & ((1u << s) - 1u));
}

// Stages [b0, b1) of a window at s on the 16 registers of one lane.
__device__ __forceinline__ void run_window(int64_t (&xr)[16], int64_t (&xi)[16], const int64_t *__restrict__ tw,
                                           uint32_t t, int s, int b0, int b1, int logn) {
    for (int b = b0; b < b1; ++b) {
        const int rb = b - s;   // register bit of this stage
        const uint32_t half_mask = (1u << b) - 1u;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (r & (1 << rb)) continue;
            const int q = r | (1 << rb);
            int64_t wr = 0, wi = 0;
            if (b > 0) {
                const uint32_t k = (win_pos(t, r, s) & half_mask) << (logn - 1 - b);
                wr = tw[2 * k], wi = tw[2 * k + 1];
            }
            butterfly(xr[r], xi[r], xr[q], xi[q], wr, wi, b == 0);
        }
    }
}

// ---------------------------------------------------------------- n <= 16
// One thread per FFT; registers indexed by position.
template <int LOGN>
__global__ __launch_bounds__(256) void fft_small_kernel(int64_t *__restrict__ re, int64_t *__restrict__ im,
                                                        const int64_t *__restrict__ tw, int64_t batch) {
    constexpr int N = 1 << LOGN;
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= batch) return;
    int64_t *R = re + f * N, *I = im + f * N;
    int64_t xr[N], xi[N];
#pragma unroll
    for (int p = 0; p < N; ++p) {
        const uint32_t src = bitrev((uint32_t)p, LOGN);
        xr[p] = R[src], xi[p] = I[src];
    }
#pragma unroll
    for (int b = 0; b < LOGN; ++b)
#pragma unroll
        for (int p = 0; p < N; ++p) {
            if (p & (1 << b)) continue;
            int64_t wr = 0, wi = 0;
            if (b > 0) {
                const int k = (p & ((1 << b) - 1)) << (LOGN - 1 - b);
                wr = tw[2 * k], wi = tw[2 * k + 1];
            }
            butterfly(xr[p], xi[p], xr[p | (1 << b)], xi[p | (1 << b)], wr, wi, b == 0);
        }
#pragma unroll
    for (int p = 0; p < N; ++p) R[p] = xr[p], I[p] = xi[p];
}

// ---------------------------------------------------------------- 32 <= n <= 2048
// L = n / 16 lanes per FFT, 256 / L FFTs per 256-thread block, a block-
// uniform grid-stride loop over the batch.  LDS holds one component of every
// FFT of the block at a time (index pos + pos / 16: one pad int64 per 16, so
// the 16 lanes of a window write 16 distinct bank pairs).
template <int LOGN>
__global__ __launch_bounds__(256) void fft_lds_kernel(int64_t *__restrict__ re, int64_t *__restrict__ im,
                                                      const int64_t *__restrict__ tw, int64_t batch) {
    constexpr int N = 1 << LOGN, L = N / 16, FPB = 256 / L, NP = (LOGN + 3) / 4;
    constexpr int STRIDE = N + N / 16;
    static_assert(LOGN >= 5 && LOGN <= 11, "LDS FFT size");
    __shared__ int64_t sm[FPB * STRIDE];
    const int f = threadIdx.x / L;
    const uint32_t t = threadIdx.x % L;
    int64_t *smf = sm + f * STRIDE;
    for (int64_t f0 = (int64_t)blockIdx.x * FPB; f0 < batch; f0 += (int64_t)gridDim.x * FPB) {
        const int64_t fi = f0 + f;
        const bool live = fi < batch;
        int64_t *R = re + (live ? fi : 0) * N, *I = im + (live ? fi : 0) * N;
        int64_t xr[16], xi[16];
        // window 0 (s = 0): position 16 t + r holds x[bitrev(16 t + r)]
        const uint32_t tb = bitrev(t, LOGN - 4);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t src = (bitrev((uint32_t)r, 4) << (LOGN - 4)) | tb;
            xr[r] = live ? R[src] : 0;
            xi[r] = live ? I[src] : 0;
        }
        run_window(xr, xi, tw, t, 0, 0, 4, LOGN);
#pragma unroll
        for (int p = 1; p < NP; ++p) {
            const int sp = 4 * (p - 1) < LOGN - 4 ? 4 * (p - 1) : LOGN - 4;   // previous window
            const int s = 4 * p < LOGN - 4 ? 4 * p : LOGN - 4;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                int64_t(&x)[16] = c ? xi : xr;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t pos = win_pos(t, r, sp);
                    smf[pos + (pos >> 4)] = x[r];
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t pos = win_pos(t, r, s);
                    x[r] = smf[pos + (pos >> 4)];
                }
                __syncthreads();
            }
            run_window(xr, xi, tw, t, s, 4 * p, 4 * p + 4 < LOGN ? 4 * p + 4 : LOGN, LOGN);
        }
        if (live) {
            const int s = 4 * (NP - 1) < LOGN - 4 ? 4 * (NP - 1) : LOGN - 4;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t pos = win_pos(t, r, s);
                R[pos] = xr[r], I[pos] = xi[r];
            }
        }
    }
}

// ---------------------------------------------------------------- n >= 4096
// One pass = the stages of one 4-bit window, global memory to global memory.
// The first pass reads through the bit reversal.  Thread g: FFT g / (n/16),
// lane-group index t = g % (n/16).
__global__ __launch_bounds__(256) void fft_pass_kernel(const int64_t *__restrict__ sre, const int64_t *__restrict__ sim,
                                                       int64_t *__restrict__ dre, int64_t *__restrict__ dim,
                                                       const int64_t *__restrict__ tw, int logn, int s, int b0, int b1,
                                                       bool first, int64_t batch) {
    const int64_t n = (int64_t)1 << logn, groups = n >> 4;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (g >= batch * groups) return;
    const int64_t fi = g / groups;
    const uint32_t t = (uint32_t)(g % groups);
    const int64_t off = fi * n;
    int64_t xr[16], xi[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t pos = win_pos(t, r, s);
        const uint32_t src = first ? bitrev(pos, logn) : pos;
        xr[r] = sre[off + src], xi[r] = sim[off + src];
    }
    run_window(xr, xi, tw, t, s, b0, b1, logn);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t pos = win_pos(t, r, s);
        dre[off + pos] = xr[r], dim[off + pos] = xi[r];
    }
}

__global__ void copy_i64_kernel(const int64_t *__restrict__ src, int64_t *__restrict__ dst, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}

}  // namespace fft

size_t fft_workspace_bytes(int logn, int64_t batch) {
    if (logn <= 11) return 0;
    return 2 * (size_t)batch * ((size_t)1 << logn) * sizeof(int64_t);
}

// batch transforms of n = 2^logn points, transform f at re + f n / im + f n,
// in place.  logn in [0, 30]; ws: fft_workspace_bytes(logn, batch) bytes.
hipError_t launch_fft_q16(int64_t *re, int64_t *im, const int64_t *tw, int logn, int64_t batch, void *ws,
                          hipStream_t s) {
    using namespace fft;
    if (batch <= 0) return hipSuccess;
    if (logn < 0 || logn > 30) return hipErrorInvalidValue;
    const int64_t n = (int64_t)1 << logn;
    const unsigned cap = 256 * 16;   // resident-size grid for the grid-stride kernels
    switch (logn) {
#define SMALL(LG) \
    case LG: hipLaunchKernelGGL(fft_small_kernel<LG>, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s, re, im, tw, batch); break;
    SMALL(0) SMALL(1) SMALL(2) SMALL(3) SMALL(4)
#undef SMALL
#define LDS(LG)                                                                                                 \
    case LG: {                                                                                                  \
        const int64_t fpb = 256 / ((1 << LG) / 16), blocks = (batch + fpb - 1) / fpb;                         \
        hipLaunchKernelGGL(fft_lds_kernel<LG>, dim3((unsigned)(blocks < cap ? blocks : cap)), dim3(256), 0, s, re, im, tw, \
                           batch);                                                                              \
        break;                                                                                                  \
    }
    LDS(5) LDS(6) LDS(7) LDS(8) LDS(9) LDS(10) LDS(11)
#undef LDS
    default: {
        if (!ws) return hipErrorInvalidValue;
        int64_t *wre = (int64_t *)ws, *wim = wre + batch * n;
        const int np = (logn + 3) / 4;
        const int64_t threads = batch * (n >> 4);
        const dim3 grid((unsigned)((threads + 255) / 256));
        // passes alternate buffers; an odd count ends in the workspace
        int64_t *src_re = re, *src_im = im;
        for (int p = 0; p < np; ++p) {
            const int sw = 4 * p < logn - 4 ? 4 * p : logn - 4;
            const int b1 = 4 * p + 4 < logn ? 4 * p + 4 : logn;
            int64_t *dst_re = (p % 2 == 0) ? wre : re, *dst_im = (p % 2 == 0) ? wim : im;
            hipLaunchKernelGGL(fft_pass_kernel, grid, dim3(256), 0, s, src_re, src_im, dst_re, dst_im, tw, logn, sw,
                               4 * p, b1, p == 0, batch);
            src_re = dst_re, src_im = dst_im;
        }
        if (src_re != re) {
            const int64_t cnt = batch * n;
            const unsigned gb = (unsigned)((cnt + 255) / 256 < cap ? (cnt + 255) / 256 : cap);
            hipLaunchKernelGGL(copy_i64_kernel, dim3(gb), dim3(256), 0, s, wre, re, cnt);
            hipLaunchKernelGGL(copy_i64_kernel, dim3(gb), dim3(256), 0, s, wim, im, cnt);
        }
        break;
    }
    }
    return hipGetLastError();
}

}  // namespace det
