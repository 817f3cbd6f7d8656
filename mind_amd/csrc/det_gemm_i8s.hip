// det_gemm_i8s.hip -- int8 GEMM for tiny shapes: one launch, no workspace,
// v_dot4_i32_i8 on the VALU.
//
// Semantics (reference src/mlir/lowering.rs:8371-9265, oracle
// benches/det_matmul_i8.rs:232-245):
//     C[i,j] = (int32) sum_k A[i,k] * B[k,j]      (exact, wrapped mod 2^32)
// v_dot4_i32_i8 without clamping adds four int8 products to an int32 with
// the same wrap, and integer addition is associative, so any grouping of
// the terms gives the reference's bits.
//
// The MFMA kernels (det_gemm_i8.hip) stage 128- or 256-row tiles through a
// multi-step DMA pipeline; below one such tile (the reference bench's own
// 16^3 and 64^3, M or N under 128) that pipeline's prologue and the 256x256
// edge kernel's masked epilogue are the whole cost.  Here one 1024-thread
// workgroup owns a 16x16 output tile: four K slices of 256 threads, one
// output per thread in each, walk K in chunks of KC bytes staged through
// LDS (A rows as [16][KC], B as its transpose [16][KC], so both operands of
// a thread's dot products are K-contiguous 16-byte reads; the padded row
// stride spreads the 16 columns' reads over all 64 banks); the four slices'
// sums meet in LDS at the end.  Operands are staged with byte buffer loads,
// invalid elements at an out-of-range offset (read as zero, and a zero
// product adds nothing), so any alignment and any K, N are taken as they
// are: no repacking.  The router (i8_small) sends a shape here only while
// its tiles fit one round of the compute units and K stays short.
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace i8s {

constexpr int TM = 16, TN = 16, KS = 4, KC = 256, LDK = KC + 16, THREADS = TM * TN * KS;
constexpr int SLICE = KC / KS;   // k per slice and chunk

__device__ __forceinline__ uint32_t load_b8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}

// A is [M][K], B is [K][N], both int8 row-major; M * K and K * N below 2^31.
__global__ __launch_bounds__(THREADS) void small_kernel(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                       int32_t *__restrict__ C, int M, int N, int K, int tiles_n) {
    __shared__ __attribute__((aligned(16))) uint8_t sA[TM][LDK];
    __shared__ __attribute__((aligned(16))) uint8_t sB[TN][LDK];   // sB[c][k] = B[k][n0 + c]
    const int t = threadIdx.x, o = t & 255, ks = t >> 8;
    const int m0 = (blockIdx.x / tiles_n) * TM, n0 = (blockIdx.x % tiles_n) * TN;
    const int r = o >> 4, c = o & 15;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)K * (uint32_t)N);
    // staging roles: 4 consecutive k of one A row, and 4 consecutive k of
    // one B column (consecutive threads take consecutive columns)
    const int ar = t >> 6, ak = (t & 63) * 4;
    const int bc = t & 15, bk = (t >> 4) * 4;
    int32_t acc = 0;
    for (int k0 = 0; k0 < K; k0 += KC) {
        uint32_t va[4], vb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gm = m0 + ar, gk = k0 + ak + j;
            va[j] = load_b8(ra, gm < M && gk < K ? (uint32_t)gm * (uint32_t)K + (uint32_t)gk : OOB_OFFSET);
            const int gn = n0 + bc, gk2 = k0 + bk + j;
            vb[j] = load_b8(rb, gn < N && gk2 < K ? (uint32_t)gk2 * (uint32_t)N + (uint32_t)gn : OOB_OFFSET);
        }
        *(uint32_t *)&sA[ar][ak] = va[0] | va[1] << 8 | va[2] << 16 | va[3] << 24;
        *(uint32_t *)&sB[bc][bk] = vb[0] | vb[1] << 8 | vb[2] << 16 | vb[3] << 24;
        __syncthreads();
        const int kb = ks * SLICE, kn = min(SLICE, K - k0 - kb);   // this slice's k range in the chunk
        for (int k = 0; k < kn; k += 16) {   // past K the chunk holds zeros
            const int4 a = *(const int4 *)&sA[r][kb + k];
            const int4 b = *(const int4 *)&sB[c][kb + k];
            acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
            acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
            acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
            acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
        }
        __syncthreads();
    }
    // the four slices' sums (mod 2^32, any order) through the free A stage
    int32_t *part = (int32_t *)&sA[0][0];
    if (ks > 0) part[(ks - 1) * 256 + o] = acc;
    __syncthreads();
    if (ks == 0) {
        acc = (int32_t)((uint32_t)acc + (uint32_t)part[o] + (uint32_t)part[256 + o] + (uint32_t)part[512 + o]);
        const int gm = m0 + r, gn = n0 + c;
        if (gm < M && gn < N) C[(size_t)gm * N + gn] = acc;
    }
}

}  // namespace i8s

// The MFMA kernels win once their tiles have work to pipeline: over more
// than one round of 16x16 tiles (512^3: 4.6 us there, 9.0 here), and for
// K > 512 on shapes their full 128-row tiles take (128x1024x128: 5.3 against
// 6.4 us).  Other shapes would go to the edge or byte-load kernels or be
// repacked first, which costs more up to K = 4096 (16x4096x16: 38 against
// 20 us; 300x1000x77: 13.3 against 7.5 us).
bool i8_small(int M, int N, int K) {
    if (K < 1) return false;
    const long long tiles = (long long)((M + i8s::TM - 1) / i8s::TM) * ((N + i8s::TN - 1) / i8s::TN);
    if (tiles > cu_count()) return false;
    const bool mfma_tiles = M % 128 == 0 && N % 128 == 0 && K % 128 == 0;
    return K <= (mfma_tiles ? I8_SMALL_K : I8_SMALL_K_ODD);
}

hipError_t launch_gemm_i8_small(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, hipStream_t s) {
    const int tiles_m = (M + i8s::TM - 1) / i8s::TM, tiles_n = (N + i8s::TN - 1) / i8s::TN;
    hipLaunchKernelGGL(i8s::small_kernel, dim3(tiles_m * tiles_n), dim3(i8s::THREADS), 0, s, A, B, C, M, N, K,
                       tiles_n);
    return hipGetLastError();
}

}  // namespace det
