// det_gemm_q16s.hip -- Q16.16 GEMM for small shapes: one launch, no
// workspace, the per-term floor computed directly on the VALU.
//
// Semantics (reference src/mlir/lowering.rs:9300-9410, oracle
// benches/det_matmul_q16.rs:227-240):
//     C[i,j] = (int32) sum_k ( (int64)A[i,k] * (int64)B[k,j]  >>arith 16 )
// Each term's low 32 bits are bits [16, 48) of the 64-bit product, and the
// truncation to int32 keeps only the low 32 bits of the sum, so C is the sum
// mod 2^32 of those bit fields: one 64-bit product and one alignbit per term,
// accumulated in uint32 in any order.
//
// The limb-MFMA kernel (det_gemm_q16x.hip) needs an operand prep launch and
// a workspace, and on grids of a few 64x64 tiles a K-split reduction launch
// too: at the reference bench's own Q16 sweep sizes (16^3 .. 512^3) those
// launches, not the arithmetic, set the time.  Here one 1024-thread
// workgroup owns a 16x16 output tile: four K slices of 256 threads, one
// output per thread in each, walk K in chunks of KC staged through LDS (A
// rows as [16][KC], B as its transpose [16][KC], so both operands of a
// thread's terms are K-contiguous 16-byte reads, and the padded row stride
// spreads the 16 columns' reads over all 64 banks); the four slices' sums
// meet in LDS at the end.  The staging loads are buffer loads whose invalid
// elements take an out-of-range offset (returned as zero, and a zero term
// adds nothing), so they issue back to back without branches.  The cost per
// thread is K / 4 terms per round of tiles over the compute units, so the
// router (q16_small) sends a shape here only while that stays small.
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace q16s {

constexpr int TM = 16, TN = 16, KS = 4, KC = 256, LDK = KC + 4, THREADS = TM * TN * KS;
constexpr int SLICE = KC / KS;                 // k per slice and chunk
constexpr int PER = TM * KC / THREADS;         // staged elements per thread and operand

__device__ __forceinline__ uint32_t term(int32_t a, int32_t b) {
    const uint64_t p = (uint64_t)((int64_t)a * (int64_t)b);
    return __builtin_amdgcn_alignbit((uint32_t)(p >> 32), (uint32_t)p, 16);
}

// B is [K][N] (row-major), or [N][K] when BT.  M * K * 4 and K * N * 4 are
// below 2^31 (buffer offsets).
template <bool BT>
__global__ __launch_bounds__(THREADS) void small_kernel(const int32_t *__restrict__ A, const int32_t *__restrict__ B,
                                                        int32_t *__restrict__ C, int M, int N, int K, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int32_t sA[TM][LDK];
    __shared__ __attribute__((aligned(16))) int32_t sB[TN][LDK];   // sB[c][k] = B[k][n0 + c]
    const int t = threadIdx.x, o = t & 255, ks = t >> 8;
    const int m0 = (blockIdx.x / tiles_n) * TM, n0 = (blockIdx.x % tiles_n) * TN;
    const int r = o >> 4, c = o & 15;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K * 4u);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)K * (uint32_t)N * 4u);
    uint32_t acc = 0;
    for (int k0 = 0; k0 < K; k0 += KC) {
        uint32_t va[PER], vb[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = i * THREADS + t;
            const int ar = idx / KC, ak = idx % KC;   // A (and B^T): consecutive threads along K
            const int gm = m0 + ar, gk = k0 + ak;
            va[i] = buf_load4(ra, gm < M && gk < K ? ((uint32_t)gm * (uint32_t)K + (uint32_t)gk) * 4u : OOB_OFFSET);
            if (BT) {
                const int gn = n0 + ar;
                vb[i] = buf_load4(rb, gn < N && gk < K ? ((uint32_t)gn * (uint32_t)K + (uint32_t)gk) * 4u : OOB_OFFSET);
            } else {
                const int bk = idx / TN, bc = idx % TN;   // row-major B: consecutive threads along N
                const int gn = n0 + bc, gk2 = k0 + bk;
                vb[i] = buf_load4(rb, gn < N && gk2 < K ? ((uint32_t)gk2 * (uint32_t)N + (uint32_t)gn) * 4u : OOB_OFFSET);
            }
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = i * THREADS + t;
            sA[idx / KC][idx % KC] = (int32_t)va[i];
            if (BT) sB[idx / KC][idx % KC] = (int32_t)vb[i];
            else sB[idx % TN][idx / TN] = (int32_t)vb[i];
        }
        __syncthreads();
        const int kb = ks * SLICE, kn = min(SLICE, K - k0 - kb);   // this slice's k range in the chunk
        for (int k = 0; k < kn; k += 16) {   // past K the chunk holds zeros
            int4 a[4], b[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u] = *(const int4 *)&sA[r][kb + k + 4 * u];
                b[u] = *(const int4 *)&sB[c][kb + k + 4 * u];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                acc += term(a[u].x, b[u].x) + term(a[u].y, b[u].y) + term(a[u].z, b[u].z) + term(a[u].w, b[u].w);
        }
        __syncthreads();
    }
    // the four slices' sums (mod 2^32, any order) through the free A stage
    uint32_t *part = (uint32_t *)&sA[0][0];
    if (ks > 0) part[(ks - 1) * 256 + o] = acc;
    __syncthreads();
    if (ks == 0) {
        acc += part[o] + part[256 + o] + part[512 + o];
        const int gm = m0 + r, gn = n0 + c;
        if (gm < M && gn < N) C[(size_t)gm * N + gn] = (int32_t)acc;
    }
}

}  // namespace q16s

// The direct kernel costs K / 4 terms per thread and round of 16x16 tiles
// over the compute units, plus a fixed cost per workgroup; past
// Q16_SMALL_ROUNDS rounds or Q16_SMALL_TERMS of K times rounds the limb
// kernel's prep and extra launches are the cheaper overhead (measured
// crossovers: 512x1024x512, 4 rounds of K = 1024, still runs faster here;
// 1024x64x1024, 16 rounds, and 1024x256x1024 do not).  The operand sizes it
// admits stay far below the 2^31-byte buffer range.
bool q16_small(int M, int N, int K) {
    if (K < 1) return false;
    const long long tiles = (long long)((M + q16s::TM - 1) / q16s::TM) * ((N + q16s::TN - 1) / q16s::TN);
    const long long cus = cu_count(), rounds = (tiles + cus - 1) / cus;
    const long long a_bytes = 4LL * M * K, b_bytes = 4LL * K * N;
    return rounds <= Q16_SMALL_ROUNDS && rounds * K <= Q16_SMALL_TERMS && a_bytes < (1LL << 31) &&
           b_bytes < (1LL << 31);
}

hipError_t launch_gemm_q16_small(const int32_t *A, const int32_t *B, int32_t *C, int M, int N, int K, bool b_is_t,
                                 hipStream_t s) {
    const int tiles_m = (M + q16s::TM - 1) / q16s::TM, tiles_n = (N + q16s::TN - 1) / q16s::TN;
    if (b_is_t)
        hipLaunchKernelGGL(q16s::small_kernel<true>, dim3(tiles_m * tiles_n), dim3(q16s::THREADS), 0, s, A, B, C, M,
                           N, K, tiles_n);
    else
        hipLaunchKernelGGL(q16s::small_kernel<false>, dim3(tiles_m * tiles_n), dim3(q16s::THREADS), 0, s, A, B, C, M,
                           N, K, tiles_n);
    return hipGetLastError();
}

}  // namespace det
