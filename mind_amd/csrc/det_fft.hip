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
//                      a block of transforms runs in int32 when a bound on
//                      its inputs proves that every intermediate fits (same
//                      integers, cheaper products), else in int64;
//   * n >= 4096      : one global-memory pass per 4-bit window, out of place
//                      through a workspace (fft_pass_kernel).
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace fft {

// Value arithmetic.  int64_t: the general path, wrapping like MIND's i64.
// int32_t: the bounded path, only taken when every intermediate value is
// known to fit in int32 (then 32-bit arithmetic gives the same integers):
// one signed 32 x 32 -> 64 product per qmul, and the shifted product fits in
// int32 because |qmul(w, x)| <= |x| for |w| <= 2^16.
__device__ __forceinline__ int64_t vadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
__device__ __forceinline__ int64_t vsub(int64_t a, int64_t b) { return (int64_t)((uint64_t)a - (uint64_t)b); }
__device__ __forceinline__ int32_t vadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
__device__ __forceinline__ int32_t vsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
__device__ __forceinline__ int64_t qm(int64_t w, int64_t v) { return ((int64_t)((uint64_t)w * (uint64_t)v)) >> 16; }
__device__ __forceinline__ int32_t qm(int64_t w, int32_t v) {
    const int64_t p = (int64_t)(int32_t)w * (int64_t)v;
    return (int32_t)(p >> 16);
}

// One butterfly (peeled: the span-2 stage, no twiddle) on (a, b).
template <typename V>
__device__ __forceinline__ void butterfly(V &ar, V &ai, V &br, V &bi, int64_t wr, int64_t wi, bool peeled) {
    V tr, ti;
    if (peeled) {
        tr = br, ti = bi;
    } else {
        tr = vsub(qm(wr, br), qm(wi, bi));
        ti = vadd(qm(wr, bi), qm(wi, br));
    }
    const V ur = ar, ui = ai;
    ar = vadd(ur, tr), ai = vadd(ui, ti);
    br = vsub(ur, tr), bi = vsub(ui, ti);
}

// Largest input magnitude for which a 2^logn-point transform stays in int32
// when every twiddle component is within [-2^16, 2^16]: |qmul(w, x)| <= |x|,
// so a span-2 stage at most doubles the largest magnitude and each later
// stage at most triples it (|a +- (qmul - qmul)| <= 3 max).
__host__ __device__ constexpr int64_t i32_input_bound(int logn) {
    int64_t g = logn >= 1 ? 2 : 1;
    for (int i = 1; i < logn; ++i) g *= 3;
    return 2147483647LL / g;
}
constexpr int64_t TW_SMALL = 65536;

__device__ __forceinline__ uint32_t bitrev(uint32_t v, int bits) { return bits ? __brev(v) >> (32 - bits) : 0u; }

// Position of register r of lane-group index t for the window [s, s + 4).
__device__ __forceinline__ uint32_t win_pos(uint32_t t, int r, int s) {
    return ((t >> s) << (s + 4)) | ((uint32_t)r << s) | (t & ((1u << s) - 1u));
}

// Stage b = s + RB of a window at s: butterflies between registers r and
// r | 2^RB (register indices are compile-time, so the points stay in VGPRs).
template <int RB, typename V>
__device__ __forceinline__ void window_stage(V (&xr)[16], V (&xi)[16], const int64_t *__restrict__ tw,
                                             uint32_t t, int s, int logn) {
    const int b = s + RB;
    const uint32_t half_mask = (1u << b) - 1u;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (r & (1 << RB)) continue;
        constexpr int bit = 1 << RB;
        int64_t wr = 0, wi = 0;
        if (b > 0) {
            const uint32_t k = (win_pos(t, r, s) & half_mask) << (logn - 1 - b);
            wr = tw[2 * k], wi = tw[2 * k + 1];
        }
        butterfly(xr[r], xi[r], xr[r | bit], xi[r | bit], wr, wi, b == 0);
    }
}

// Stages [b0, b1) of a window at s (b0 >= s, b1 <= s + 4), in order.
template <typename V>
__device__ __forceinline__ void run_window(V (&xr)[16], V (&xi)[16], const int64_t *__restrict__ tw,
                                           uint32_t t, int s, int b0, int b1, int logn) {
    if (b0 <= s && s < b1) window_stage<0>(xr, xi, tw, t, s, logn);
    if (b0 <= s + 1 && s + 1 < b1) window_stage<1>(xr, xi, tw, t, s, logn);
    if (b0 <= s + 2 && s + 2 < b1) window_stage<2>(xr, xi, tw, t, s, logn);
    if (b0 <= s + 3 && s + 3 < b1) window_stage<3>(xr, xi, tw, t, s, logn);
}

// ---- int32 path: twiddles preloaded as int32 (valid when every component
// is within [-2^16, 2^16]).  Slot (2^rb - 1) + j of a window's table holds
// the twiddle of stage s + rb for butterflies whose register index has low
// bits j (the position bits below the stage bit are those low bits and the
// lane's own bits, so 1 + 2 + 4 + 8 slots cover a window).
struct WinTw {
    int32_t r[15], i[15];
};

template <int S, int B0, int B1, int LOGN>
__device__ __forceinline__ void load_win_tw(WinTw &w, const int64_t *__restrict__ tw, uint32_t t) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const int b = S + rb;
        if (b < B0 || b >= B1 || b == 0) continue;
#pragma unroll
        for (int j = 0; j < (1 << rb); ++j) {
            const uint32_t k = (win_pos(t, j, S) & ((1u << b) - 1u)) << (LOGN - 1 - b);
            int32_t wr = (int32_t)tw[2 * k], wi = (int32_t)tw[2 * k + 1];
            if (S == 0) {   // window 0: the same twiddles in every lane
                wr = __builtin_amdgcn_readfirstlane(wr);
                wi = __builtin_amdgcn_readfirstlane(wi);
            }
            w.r[(1 << rb) - 1 + j] = wr, w.i[(1 << rb) - 1 + j] = wi;
        }
    }
}

template <int S, int B0, int B1>
__device__ __forceinline__ void window32(int32_t (&xr)[16], int32_t (&xi)[16], const WinTw &w) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const int b = S + rb;
        if (b < B0 || b >= B1) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (r & (1 << rb)) continue;
            const int slot = (1 << rb) - 1 + (r & ((1 << rb) - 1));
            const int q = r | (1 << rb);
            butterfly(xr[r], xi[r], xr[q], xi[q], (int64_t)w.r[slot], (int64_t)w.i[slot], b == 0);
        }
    }
}

// Re-layout from window SP to window S through LDS, (re, im) as one 8-byte
// element at index pos + pos / 16.
template <int SP, int S>
__device__ __forceinline__ void transpose32(int32_t (&xr)[16], int32_t (&xi)[16], uint32_t t, uint64_t *smf) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t pos = win_pos(t, r, SP);
        smf[pos + (pos >> 4)] = (uint64_t)(uint32_t)xr[r] | ((uint64_t)(uint32_t)xi[r] << 32);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t pos = win_pos(t, r, S);
        const uint64_t v = smf[pos + (pos >> 4)];
        xr[r] = (int32_t)(uint32_t)v, xi[r] = (int32_t)(uint32_t)(v >> 32);
    }
    __syncthreads();
}

// ---------------------------------------------------------------- n <= 16
// One thread per FFT; registers indexed by position.
template <int LOGN>
__global__ __launch_bounds__(256) void fft_small_kernel(const int64_t *__restrict__ sre,
                                                        const int64_t *__restrict__ sim, int64_t *__restrict__ dre,
                                                        int64_t *__restrict__ dim, const int64_t *__restrict__ tw,
                                                        int64_t batch) {
    constexpr int N = 1 << LOGN;
    const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (f >= batch) return;
    const int64_t *R = sre + f * N, *I = sim + f * N;
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
    for (int p = 0; p < N; ++p) dre[f * N + p] = xr[p], dim[f * N + p] = xi[p];
}

// ---------------------------------------------------------------- 32 <= n <= 2048
// L = n / 16 lanes per FFT, 256 / L FFTs per 256-thread block, a block-
// uniform grid-stride loop over the batch.  Reads src, writes dst (equal for
// in place: a lane group holds its whole transform before storing).  LDS
// holds one component of every FFT of the block at a time, index
// pos + pos / 16 (one pad element per 16, so the 16 lanes of a window hit
// distinct banks).  Per block of transforms the path is chosen once, block-
// uniformly (the LDS transposes need the whole block): int32 when the table
// is small and every loaded value is within i32_input_bound, else int64.
template <int LOGN, typename V>
__device__ __forceinline__ void lds_transform(V (&xr)[16], V (&xi)[16], const int64_t *__restrict__ tw, uint32_t t,
                                              V *smf) {
    constexpr int N = 1 << LOGN, NP = (LOGN + 3) / 4;
    run_window(xr, xi, tw, t, 0, 0, 4, LOGN);
#pragma unroll
    for (int p = 1; p < NP; ++p) {
        const int sp = 4 * (p - 1) < LOGN - 4 ? 4 * (p - 1) : LOGN - 4;   // previous window
        const int s = 4 * p < LOGN - 4 ? 4 * p : LOGN - 4;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            V(&x)[16] = c ? xi : xr;
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
    (void)N;
}

// A block handles FPB transforms at a time ("group" f0 .. f0 + FPB - 1);
// lane t of slot f loads window 0 of transform f0 + f.
template <int LOGN>
__device__ __forceinline__ bool load_group(const int64_t *__restrict__ sre, const int64_t *__restrict__ sim,
                                           int64_t fi, bool live, uint32_t t, int64_t (&xr)[16], int64_t (&xi)[16]) {
    constexpr int N = 1 << LOGN;
    constexpr int64_t BOUND = i32_input_bound(LOGN);
    const int64_t off = (live ? fi : 0) * N;
    // window 0 (s = 0): position 16 t + r holds x[bitrev(16 t + r)]
    const uint32_t tb = bitrev(t, LOGN - 4);
    bool fits = true;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t src = (bitrev((uint32_t)r, 4) << (LOGN - 4)) | tb;
        xr[r] = live ? __builtin_nontemporal_load(sre + off + src) : 0;   // each point is read once
        xi[r] = live ? __builtin_nontemporal_load(sim + off + src) : 0;
        fits = fits && xr[r] >= -BOUND && xr[r] <= BOUND && xi[r] >= -BOUND && xi[r] <= BOUND;
    }
    return fits;
}

template <int LOGN, typename V>
__device__ __forceinline__ void store_group(int64_t *__restrict__ dre, int64_t *__restrict__ dim, int64_t fi,
                                            uint32_t t, const V (&xr)[16], const V (&xi)[16]) {
    constexpr int N = 1 << LOGN, NP = (LOGN + 3) / 4;
    constexpr int S_LAST = 4 * (NP - 1) < LOGN - 4 ? 4 * (NP - 1) : LOGN - 4;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t pos = win_pos(t, r, S_LAST);
        __builtin_nontemporal_store((int64_t)xr[r], dre + fi * N + pos);   // streamed: read by no one here
        __builtin_nontemporal_store((int64_t)xi[r], dim + fi * N + pos);
    }
}

// A block of transforms whose inputs are all within i32_input_bound (and a
// table within [-2^16, 2^16]) runs in int32; any other block runs the int64
// transform on the values it has already loaded (the choice is block-uniform,
// so every thread takes the same path through the LDS transposes).
template <int LOGN>
__global__ __launch_bounds__(256) void fft_lds_kernel(const int64_t *__restrict__ sre, const int64_t *__restrict__ sim,
                                                      int64_t *__restrict__ dre, int64_t *__restrict__ dim,
                                                      const int64_t *__restrict__ tw, int64_t batch) {
    constexpr int N = 1 << LOGN, L = N / 16, FPB = 256 / L, NP = (LOGN + 3) / 4;
    constexpr int STRIDE = N + N / 16;
    constexpr int S1 = 4 < LOGN - 4 ? 4 : LOGN - 4, S2 = 8 < LOGN - 4 ? 8 : LOGN - 4;
    static_assert(LOGN >= 5 && LOGN <= 11, "LDS FFT size");
    __shared__ uint64_t sm[FPB * STRIDE];
    const int f = threadIdx.x / L;
    const uint32_t t = threadIdx.x % L;
    // every twiddle component within [-2^16, 2^16] (the standard table is)
    bool small = true;
    for (int i = threadIdx.x; i < N; i += 256) {
        const int64_t w = tw[i];
        small = small && w >= -TW_SMALL && w <= TW_SMALL;
    }
    const bool tw_small = __syncthreads_and(small);
    WinTw w0, w1, w2;
    if (tw_small) {
        load_win_tw<0, 0, 4, LOGN>(w0, tw, t);
        if constexpr (NP > 1) load_win_tw<S1, 4, (8 < LOGN ? 8 : LOGN), LOGN>(w1, tw, t);
        if constexpr (NP > 2) load_win_tw<S2, 8, LOGN, LOGN>(w2, tw, t);
    }
    uint64_t *smf = sm + f * STRIDE;
    for (int64_t f0 = (int64_t)blockIdx.x * FPB; f0 < batch; f0 += (int64_t)gridDim.x * FPB) {
        const int64_t fi = f0 + f;
        const bool live = fi < batch;
        int64_t xr[16], xi[16];
        const bool fits = load_group<LOGN>(sre, sim, fi, live, t, xr, xi);
        if (!__syncthreads_and(fits && tw_small)) {
            lds_transform<LOGN>(xr, xi, tw, t, (int64_t *)smf);
            if (live) store_group<LOGN>(dre, dim, fi, t, xr, xi);
            continue;
        }
        int32_t yr[16], yi[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) yr[r] = (int32_t)xr[r], yi[r] = (int32_t)xi[r];
        window32<0, 0, 4>(yr, yi, w0);
        if constexpr (NP > 1) {
            transpose32<0, S1>(yr, yi, t, smf);
            window32<S1, 4, (8 < LOGN ? 8 : LOGN)>(yr, yi, w1);
        }
        if constexpr (NP > 2) {
            transpose32<S1, S2>(yr, yi, t, smf);
            window32<S2, 8, LOGN>(yr, yi, w2);
        }
        if (live) store_group<LOGN>(dre, dim, fi, t, yr, yi);
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

// A few transforms (batch <= FEW_BATCH, 32 <= n <= 2048): one workgroup per
// transform, its points and the twiddle table in LDS, and one butterfly per
// thread and stage, so the latency of a lone call is logn barrier-separated
// stages instead of a lane walking its 16 points through every stage (the
// batched kernel gives a single transform only n / 16 lanes).  Same
// butterflies, same stage order: same bits.  Loads and stores touch each
// point once (an in-place call reads all of its transform before writing, at
// the first barrier).  Measured against the batched kernel (device time,
// same box): 256 points x1 8.1 -> 4.0 us, x512 9.4 -> 5.3; 2048 points x1
// 17.0 -> 11.3, x64 19.7 -> 11.7; past 512 transforms the batched kernel's
// throughput wins (256 points x2048: 9.8 against 14.0 us).
constexpr int FEW_BATCH = 512;

__global__ __launch_bounds__(1024) void fft_few_kernel(const int64_t *__restrict__ sre, const int64_t *__restrict__ sim,
                                                       int64_t *dre, int64_t *dim, const int64_t *__restrict__ tw,
                                                       int logn) {
    __shared__ int64_t lre[2048], lim[2048], ltw[2048];
    const int n = 1 << logn, half_n = n >> 1, t = threadIdx.x;
    const size_t base = (size_t)blockIdx.x * n;
    for (int i = t; i < n; i += blockDim.x) {   // bit reversal on the way in
        const uint32_t p = bitrev((uint32_t)i, logn);
        lre[p] = sre[base + i];
        lim[p] = sim[base + i];
        ltw[i] = tw[i];                          // the table is read once, then from LDS
    }
    __syncthreads();
    for (int b = 0; b < logn; ++b) {   // stage b pairs positions that differ in bit b
        const int h = 1 << b;
        for (int q = t; q < half_n; q += blockDim.x) {
            const int j = q & (h - 1), ia = ((q >> b) << (b + 1)) | j, ib = ia + h;
            int64_t wr = 0, wi = 0;
            if (b > 0) {
                const int k = j << (logn - 1 - b);
                wr = ltw[2 * k], wi = ltw[2 * k + 1];
            }
            int64_t ar = lre[ia], ai = lim[ia], br = lre[ib], bi = lim[ib];
            butterfly(ar, ai, br, bi, wr, wi, b == 0);
            lre[ia] = ar, lim[ia] = ai, lre[ib] = br, lim[ib] = bi;
        }
        __syncthreads();
    }
    for (int i = t; i < n; i += blockDim.x) {
        dre[base + i] = lre[i];
        dim[base + i] = lim[i];
    }
}

}  // namespace fft

size_t fft_workspace_bytes(int logn, int64_t batch) {
    if (logn <= 11) return 0;
    return 2 * (size_t)batch * ((size_t)1 << logn) * sizeof(int64_t);
}

// batch transforms of n = 2^logn points: transform f read from sre / sim
// + f n and written to dre / dim + f n (the same pointers for in place).
// logn in [0, 30]; ws: fft_workspace_bytes(logn, batch) bytes.
hipError_t launch_fft_q16(const int64_t *sre, const int64_t *sim, int64_t *dre, int64_t *dim, const int64_t *tw,
                          int logn, int64_t batch, void *ws, hipStream_t s) {
    using namespace fft;
    if (batch <= 0) return hipSuccess;
    if (logn < 0 || logn > 30) return hipErrorInvalidValue;
    const int64_t n = (int64_t)1 << logn;
    const unsigned cap = 256 * 16;   // resident-size grid for the grid-stride kernels
    switch (logn) {
#define SMALL(LG)                                                                                              \
    case LG:                                                                                                   \
        hipLaunchKernelGGL(fft_small_kernel<LG>, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s, sre, sim, \
                           dre, dim, tw, batch);                                                               \
        break;
    SMALL(0) SMALL(1) SMALL(2) SMALL(3) SMALL(4)
#undef SMALL
#define LDS(LG)                                                                                                \
    case LG: {                                                                                                 \
        if (batch <= FEW_BATCH) {                                                                              \
            const unsigned threads = (1u << LG) / 2 < 1024 ? (1u << LG) / 2 : 1024;                            \
            hipLaunchKernelGGL(fft_few_kernel, dim3((unsigned)batch), dim3(threads), 0, s, sre, sim, dre, dim, tw, \
                               LG);                                                                            \
            break;                                                                                             \
        }                                                                                                      \
        const int64_t fpb = 256 / ((1 << LG) / 16), blocks = (batch + fpb - 1) / fpb;                        \
        const unsigned grid = (unsigned)(blocks < cap ? blocks : cap);                                         \
        hipLaunchKernelGGL(fft_lds_kernel<LG>, dim3(grid), dim3(256), 0, s, sre, sim, dre, dim, tw, batch);   \
        break;                                                                                                 \
    }
    LDS(5) LDS(6) LDS(7) LDS(8) LDS(9) LDS(10) LDS(11)
#undef LDS
    default: {
        if (!ws) return hipErrorInvalidValue;
        int64_t *wre = (int64_t *)ws, *wim = wre + batch * n;
        const int np = (logn + 3) / 4;
        const int64_t threads = batch * (n >> 4);
        const dim3 grid((unsigned)((threads + 255) / 256));
        // pass 0 reads the source through the bit reversal into the
        // workspace; later passes alternate dst and workspace; an odd pass
        // count ends in the workspace and is copied to dst
        const int64_t *src_re = sre, *src_im = sim;
        for (int p = 0; p < np; ++p) {
            const int sw = 4 * p < logn - 4 ? 4 * p : logn - 4;
            const int b1 = 4 * p + 4 < logn ? 4 * p + 4 : logn;
            int64_t *to_re = (p % 2 == 0) ? wre : dre, *to_im = (p % 2 == 0) ? wim : dim;
            hipLaunchKernelGGL(fft_pass_kernel, grid, dim3(256), 0, s, src_re, src_im, to_re, to_im, tw, logn, sw,
                               4 * p, b1, p == 0, batch);
            src_re = to_re, src_im = to_im;
        }
        if (src_re == wre) {
            const int64_t cnt = batch * n;
            const unsigned gb = (unsigned)((cnt + 255) / 256 < cap ? (cnt + 255) / 256 : cap);
            hipLaunchKernelGGL(copy_i64_kernel, dim3(gb), dim3(256), 0, s, wre, dre, cnt);
            hipLaunchKernelGGL(copy_i64_kernel, dim3(gb), dim3(256), 0, s, wim, dim, cnt);
        }
        break;
    }
    }
    return hipGetLastError();
}

}  // namespace det
