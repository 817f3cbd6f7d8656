// det_gemm_small.hip -- int8 and int16 GEMMs for tiny shapes: one launch,
// no workspace, v_dot4_i32_i8 / v_dot2_i32_i16 on the VALU.
//
// Semantics (reference src/mlir/lowering.rs:8371-9265 and the int16 GEMM
// of benches/det_matmul_i16.rs:218-230; oracles benches/det_matmul_i8.rs:
// 232-245 and det_matmul_i16.rs):
//     C[i,j] = (int32) sum_k A[i,k] * B[k,j]      (exact, wrapped mod 2^32)
// v_dot4_i32_i8 and v_dot2_i32_i16 without clamping add four int8 / two
// int16 products to an int32 with the same wrap, and integer addition is
// associative, so any grouping of the terms gives the reference's bits.
//
// The MFMA kernels (det_gemm_i8.hip, and the int16 GEMM as an int8 GEMM on
// limb-interleaved operands, det_gemm_i16x.hip) stage 128- or 256-row tiles
// through a multi-step DMA pipeline, after an operand prep launch for
// int16; below one such tile (the reference bench's own int8 16^3 and 64^3,
// M or N under 128) that pipeline's prologue, the 256x256 edge kernel's
// masked epilogue and the prep are the whole cost.  Here one 1024-thread
// workgroup owns a 16x16 output tile: four K slices of 256 threads, one
// output per thread in each, walk K in chunks of KC elements (256 bytes per
// row) staged through LDS (A rows as [16][KC], B as its transpose [16][KC],
// so both operands of a thread's dot products are K-contiguous 16-byte
// reads; the padded row stride spreads the 16 columns' reads over all 64
// banks); the four slices' sums meet in LDS at the end.  Operands are staged
// with element-wide buffer loads, invalid elements at an out-of-range offset
// (read as zero, and a zero product adds nothing), so any alignment and any
// K, N are taken as they are: no repacking.  The routers (i8_small,
// i16_small) send a shape here only while its tiles fit one round of the
// compute units and K stays short.
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace tiny {

constexpr int TM = 16, TN = 16, KS = 4, ROWB = 256, LDB = ROWB + 16, THREADS = TM * TN * KS;

// One int8 or int16 element by buffer load, zero-extended into a dword.
template <typename T>
__device__ __forceinline__ uint32_t load_elem(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (sizeof(T) == 1) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
    else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// acc + the dot product of the packed elements of one dword of each operand.
template <typename T>
__device__ __forceinline__ int32_t dot(int32_t a, int32_t b, int32_t acc) {
    if constexpr (sizeof(T) == 1) return __builtin_amdgcn_sdot4(a, b, acc, false);
    else return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b), acc, false);
}

// A is [M][K], B is [K][N], both T row-major; M * K and K * N bytes below
// 2^31.
template <typename T>
__global__ __launch_bounds__(THREADS) void small_kernel(const T *__restrict__ A, const T *__restrict__ B,
                                                       int32_t *__restrict__ C, int M, int N, int K, int tiles_n) {
    constexpr int ES = sizeof(T), KC = ROWB / ES, SLICE = KC / KS, PER = 4 / ES;   // PER elements per dword
    __shared__ __attribute__((aligned(16))) uint8_t sA[TM][LDB];
    __shared__ __attribute__((aligned(16))) uint8_t sB[TN][LDB];   // sB[c] = column n0 + c of B, K-contiguous
    const int t = threadIdx.x, o = t & 255, ks = t >> 8;
    const int m0 = (blockIdx.x / tiles_n) * TM, n0 = (blockIdx.x % tiles_n) * TN;
    const int r = o >> 4, c = o & 15;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K * ES);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)K * (uint32_t)N * ES);
    // staging roles: one dword (PER consecutive k) of one A row, and one of
    // one B column (consecutive threads take consecutive columns)
    const int ar = t >> 6, ak = (t & 63) * PER;
    const int bc = t & 15, bk = (t >> 4) * PER;
    int32_t acc = 0;
    for (int k0 = 0; k0 < K; k0 += KC) {
        uint32_t wa = 0, wb = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int gm = m0 + ar, gk = k0 + ak + j;
            const uint32_t va =
                load_elem<T>(ra, gm < M && gk < K ? ((uint32_t)gm * (uint32_t)K + (uint32_t)gk) * ES : OOB_OFFSET);
            const int gn = n0 + bc, gk2 = k0 + bk + j;
            const uint32_t vb =
                load_elem<T>(rb, gn < N && gk2 < K ? ((uint32_t)gk2 * (uint32_t)N + (uint32_t)gn) * ES : OOB_OFFSET);
            wa |= va << (8 * ES * j);
            wb |= vb << (8 * ES * j);
        }
        *(uint32_t *)&sA[ar][ak * ES] = wa;
        *(uint32_t *)&sB[bc][bk * ES] = wb;
        __syncthreads();
        const int kb = ks * SLICE, kn = min(SLICE, K - k0 - kb);   // this slice's k range in the chunk
        for (int k = 0; k < kn; k += 4 * PER) {   // 16 bytes per step; past K the chunk holds zeros
            const int4 a = *(const int4 *)&sA[r][(kb + k) * ES];
            const int4 b = *(const int4 *)&sB[c][(kb + k) * ES];
            acc = dot<T>(a.x, b.x, acc);
            acc = dot<T>(a.y, b.y, acc);
            acc = dot<T>(a.z, b.z, acc);
            acc = dot<T>(a.w, b.w, acc);
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

}  // namespace tiny

static long long small_tiles(int M, int N) {
    return (long long)((M + tiny::TM - 1) / tiny::TM) * ((N + tiny::TN - 1) / tiny::TN);
}

// The MFMA kernels win once their tiles have work to pipeline: over more
// than one round of 16x16 tiles (512^3: 4.6 us there, 9.0 here), and for
// K > 512 on shapes their full 128-row tiles take (128x1024x128: 5.3 against
// 6.4 us).  Other shapes would go to the edge or byte-load kernels or be
// repacked first, which costs more up to K = 4096 (16x4096x16: 38 against
// 20 us; 300x1000x77: 13.3 against 7.5 us).
bool i8_small(int M, int N, int K) {
    if (K < 1 || small_tiles(M, N) > cu_count()) return false;
    const bool mfma_tiles = M % 128 == 0 && N % 128 == 0 && K % 128 == 0;
    return K <= (mfma_tiles ? I8_SMALL_K : I8_SMALL_K_ODD);
}

hipError_t launch_gemm_i8_small(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, hipStream_t s) {
    const int tiles_n = (N + tiny::TN - 1) / tiny::TN;
    hipLaunchKernelGGL(tiny::small_kernel<int8_t>, dim3((unsigned)small_tiles(M, N)), dim3(tiny::THREADS), 0, s, A, B,
                       C, M, N, K, tiles_n);
    return hipGetLastError();
}

// int16: the alternative is an operand prep launch plus the interleaved
// MFMA GEMM, which on one round of 16x16 tiles costs more up to K = 4096
// (measured, same box: 16^3 8.8 against 3.5 us, 256^3 11.2 against 3.8-4.6,
// 255x2048x255 33.5 against 17.4, 16x4096x16 50 against 28).
bool i16_small(int M, int N, int K) {
    if (K < 1 || small_tiles(M, N) > cu_count()) return false;
    return K <= I16_SMALL_K;
}

hipError_t launch_gemm_i16_small(const int16_t *A, const int16_t *B, int32_t *C, int M, int N, int K,
                                 hipStream_t s) {
    const int tiles_n = (N + tiny::TN - 1) / tiny::TN;
    hipLaunchKernelGGL(tiny::small_kernel<int16_t>, dim3((unsigned)small_tiles(M, N)), dim3(tiny::THREADS), 0, s, A, B,
                       C, M, N, K, tiles_n);
    return hipGetLastError();
}

}  // namespace det
