// det_gemm_i8.hip -- exact int8 GEMM on gfx950 int8 MFMA.
//
//   C[i,j] = (int32) sum_k A[i,k] * B[k,j]        A: MxK int8 row-major
//                                                  B: KxN int8 row-major
//                                                  C: MxN int32 row-major
// Semantics of __mind_blas_matmul_mm_i8_v (reference: src/mlir/lowering.rs:
// 7687-7797 emit_vec_matmul_mm_i8, :8371-9265 emit_mm_i8_blocked; oracle
// benches/det_matmul_i8.rs:232-245): the exact sum, wrapped to 32 bits.
// v_mfma_i32_16x16x64_i8 accumulates exactly in i32 with two's-complement
// wrap-around, i.e. mod 2^32, which is exactly the reference's i64 sum
// truncated to i32.
//
// Tiling: one 256-thread workgroup (4 waves, 2x2) per 256x256 C tile, each
// wave owns a 128x128 sub-tile = 8x8 MFMA blocks (256 accumulator registers).
// K advances 64 bytes per step.  A tiles go global -> LDS unchanged (K is
// contiguous, which is what the MFMA operand wants).  B is row-major (N
// contiguous) but the MFMA B operand needs K-contiguous bytes per column, so
// every thread loads an 8(k) x 8(n) byte block and transposes it in registers
// with v_perm_b32 before writing it to LDS as B^T.  LDS rows are 64 bytes;
// the four 16-byte chunks of a row are XOR-swizzled by (row >> 1) & 3 so the
// ds_read_b128 operand fetches of 8 consecutive rows hit distinct banks.
// Two LDS buffers: the global loads for step t+1 are issued before the MFMAs
// of step t and written to the other buffer afterwards, one barrier per step.
#include "det_common.h"
#include "det_kernels.h"

namespace det {

namespace i8g {
constexpr int BM = 256, BN = 256, BK = 64, THREADS = 256;
constexpr int TILE_BYTES = BM * BK;  // == BN * BK
constexpr int GROUP_M = 4;

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

struct Frag {
    uint4 a[4];       // 4 x 16 bytes of A (rows, chunk)
    uint32_t blo[8];  // 8 rows of B, columns 0..3
    uint32_t bhi[8];  // 8 rows of B, columns 4..7
};

// Global -> registers.  FAST requires K % 16 == 0, N % 8 == 0 and 16-byte
// aligned A, 8-byte aligned B: every 16-byte A chunk and 8-byte B run is then
// either fully inside or fully outside the matrix.
template <bool FAST>
__device__ __forceinline__ void load_tile(Frag &f, const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                          int M, int N, int K, int m0, int n0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = i * THREADS + tid;
        const int row = m0 + (idx >> 2);
        const int kc = k0 + ((idx & 3) << 4);
        if (FAST) {
            if (row < M && kc < K)
                f.a[i] = *(const uint4 *)(A + (size_t)row * K + kc);
            else
                f.a[i] = make_uint4(0, 0, 0, 0);
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
            if (row < M) {
                const int8_t *p = A + (size_t)row * K;
#pragma unroll
                for (int b = 0; b < 16; ++b)
                    if (kc + b < K) w[b >> 2] |= (uint32_t)(uint8_t)p[kc + b] << ((b & 3) * 8);
            }
            f.a[i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    const int kb = tid >> 5, nb = tid & 31;
    const int nc = n0 + nb * 8;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int kr = k0 + kb * 8 + r;
        if (FAST) {
            if (kr < K && nc < N) {
                const uint2 v = *(const uint2 *)(B + (size_t)kr * N + nc);
                f.blo[r] = v.x;
                f.bhi[r] = v.y;
            } else {
                f.blo[r] = 0;
                f.bhi[r] = 0;
            }
        } else {
            uint32_t lo = 0, hi = 0;
            if (kr < K) {
                const int8_t *p = B + (size_t)kr * N;
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    if (nc + b < N) {
                        const uint32_t v = (uint32_t)(uint8_t)p[nc + b];
                        if (b < 4) lo |= v << (b * 8); else hi |= v << ((b - 4) * 8);
                    }
            }
            f.blo[r] = lo;
            f.bhi[r] = hi;
        }
    }
}

__device__ __forceinline__ void store_tile(const Frag &f, int8_t *sA, int8_t *sB, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = i * THREADS + tid;
        *(uint4 *)(sA + swz(idx >> 2, idx & 3)) = f.a[i];
    }
    uint32_t clo[8], chi[8];
    transpose8x8(f.blo, f.bhi, clo, chi);
    const int kb = tid >> 5, nb = tid & 31;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int n = nb * 8 + c;
        *(uint2 *)(sB + swz(n, kb >> 1) + ((kb & 1) << 3)) = make_uint2(clo[c], chi[c]);
    }
}

template <bool FAST>
__global__ __launch_bounds__(THREADS, 1) void gemm_i8_kernel(const int8_t *__restrict__ A,
                                                             const int8_t *__restrict__ B,
                                                             int32_t *__restrict__ C, int M, int N, int K,
                                                             int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(16))) int8_t smem[2][2][TILE_BYTES];

    const int ntiles = tiles_m * tiles_n;
    const int pid = xcd_remap(blockIdx.x, ntiles);
    const int in_group = GROUP_M * tiles_n;
    const int first_m = (pid / in_group) * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int tm = first_m + (pid % in_group) % gsize;
    const int tn = (pid % in_group) / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
    const int lr = lane & 15, lg = lane >> 4;

    v4i32 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = (v4i32){0, 0, 0, 0};

    const int nk = (K + BK - 1) / BK;
    Frag f;
    load_tile<FAST>(f, A, B, M, N, K, m0, n0, 0, tid);
    store_tile(f, smem[0][0], smem[0][1], tid);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) load_tile<FAST>(f, A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);

        const int8_t *sA = smem[cur][0];
        const int8_t *sB = smem[cur][1];
        v2i64 bf[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) bf[j] = *(const v2i64 *)(sB + swz(wn + j * 16 + lr, lg));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const v2i64 af = *(const v2i64 *)(sA + swz(wm + i * 16 + lr, lg));
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] = mfma16x16x64(af, bf[j], acc[i][j]);
        }

        if (more) store_tile(f, smem[cur ^ 1][0], smem[cur ^ 1][1], tid);
        __syncthreads();
    }

    // Epilogue: lane holds C[4*lg + r][lr] of each 16x16 block.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm + i * 16 + lg * 4 + r;
            if (row >= M) continue;
            int32_t *crow = C + (size_t)row * N;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int col = n0 + wn + j * 16 + lr;
                if (col < N) __builtin_nontemporal_store(acc[i][j][r], crow + col);
            }
        }
    }
}
}  // namespace i8g

hipError_t launch_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, hipStream_t s) {
    using namespace i8g;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const dim3 grid(tiles_m * tiles_n), block(THREADS);
    const bool fast = (K % 16 == 0) && (N % 8 == 0) && (((uintptr_t)A & 15) == 0) && (((uintptr_t)B & 7) == 0);
    if (fast)
        hipLaunchKernelGGL(gemm_i8_kernel<true>, grid, block, 0, s, A, B, C, M, N, K, tiles_m, tiles_n);
    else
        hipLaunchKernelGGL(gemm_i8_kernel<false>, grid, block, 0, s, A, B, C, M, N, K, tiles_m, tiles_n);
    return hipGetLastError();
}

}  // namespace det
