// det_gemm_i16x.hip -- int16 GEMM as one int8 MFMA GEMM on interleaved limbs.
//
// Semantics (build-defined GEMM whose every element is the reference int16
// dot, benches/det_matmul_i16.rs:218-224):
//     C[i,j] = (int32) sum_k (int64)A[i,k] * (int64)B[k,j]   (mod 2^32)
//
// With the bias identity of det_gemm_limb.hip (a = T(a) + c, c = 0x80,
// T(a) = t0 + 2^8 t1, t0 = low byte ^ 0x80 as int8, t1 = signed high byte):
//     sum_k a b = sum_{x,y} 2^(8(x+y)) sum_k t_x(a) t_y(b)
//                 + c sum_k a + c sum_k b - K c^2            (mod 2^32)
// The four limb-pair sums are the 2x2 blocks of ONE int8 GEMM
//     A2 [2M][Kp] (row 2i = t0(A row i), row 2i+1 = t1(A row i))
//   x B2 [Kp][N2] (column 2j = t0(B column j), column 2j+1 = t1(B column j))
// and B2 is simply B's bytes with each low byte XORed with 0x80.  The int8
// DMA kernel (det_gemm_i8.hip) runs that GEMM and its EPI_I16 epilogue folds
// each 2x2 block, with the bias terms, into one int32 output.  Every step is
// mod 2^32, which is the i64 sum truncated to 32 bits: no flush, any K.
//
// Prep: one launch, prep_i16 (one wave per A row: limb split, exact row
// sum; 64 x 128 tiles of B: the XOR, zero padding, up to MAX_CS exact partial
// column sums per column, added by the GEMM epilogue).
#include "det_common.h"
#include "det_kernels.h"

namespace det {

hipError_t launch_gemm_i8_i16epi(const int8_t *A2, const int8_t *B2, int M2, int N2, int Kp, const uint32_t *rowsum,
                                 const uint32_t *colsum, int ncs, int32_t *C, int M16, int N16, int K16,
                                 hipStream_t s);

namespace i16x {

// Byte mask of the valid elements of dword d of a 16-element run with nv
// valid elements (nv in [0, 16]).
__device__ __forceinline__ uint32_t valid_mask(int nv, int d) {
    const int r = nv - 4 * d;
    return r >= 4 ? 0xffffffffu : (r <= 0 ? 0u : (1u << (8 * r)) - 1u);
}

// A [M][K] int16 -> A2 [2M][Kp] int8 limb rows, rowsum [M] (mod 2^32):
// rows 4 blk .. 4 blk + 3, one wave per row.
__device__ __forceinline__ void prep_a_rows(const int16_t *__restrict__ src, int M, int K, int Kp,
                                            int8_t *__restrict__ A2, uint32_t *__restrict__ rowsum, int blk) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blk * 4 + (tid >> 6);
    if (row >= M) return;
    const int16_t *s = src + (size_t)row * K;
    uint32_t sum = 0;
    // 16 int16 (two per dword) at k0, nv of them valid -> the two limb rows
    auto emit = [&](const uint32_t (&d)[8], int k0, int nv) {
#pragma unroll
        for (int h = 0; h < 8; ++h) sum += (uint32_t)(int32_t)(int16_t)(d[h] & 0xffff) + (uint32_t)((int32_t)d[h] >> 16);
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            lo[q] = perm(d[2 * q + 1], d[2 * q], 0x06040200u) ^ (0x80808080u & valid_mask(nv, q));
            hi[q] = perm(d[2 * q + 1], d[2 * q], 0x07050301u);
        }
        *(uint4 *)(A2 + (size_t)(2 * row) * Kp + k0) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4 *)(A2 + (size_t)(2 * row + 1) * Kp + k0) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    };
    if (((K & 15) == 0) && ((((uintptr_t)src) & 15) == 0)) {
        // every 16-element chunk is full (Kp == K): up to 4 chunks per lane
        // loaded before any is processed, so 128 bytes per lane are in flight
        constexpr int U = 4;
        for (int k0 = lane * 16; k0 < K; k0 += 1024 * U) {
            uint4 v[U][2];
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (k0 + 1024 * u < K) {
                    v[u][0] = *(const uint4 *)(s + k0 + 1024 * u);
                    v[u][1] = *(const uint4 *)(s + k0 + 1024 * u + 8);
                }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (k0 + 1024 * u < K) {
                    const uint32_t d[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w,
                                           v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
                    emit(d, k0 + 1024 * u, 16);
                }
        }
    } else {
        for (int k0 = lane * 16; k0 < Kp; k0 += 1024) {
            const int nv = min(max(K - k0, 0), 16);
            uint32_t d[8];
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                const uint32_t lo = 2 * h < nv ? (uint16_t)s[k0 + 2 * h] : 0u;
                const uint32_t hi = 2 * h + 1 < nv ? (uint16_t)s[k0 + 2 * h + 1] : 0u;
                d[h] = lo | (hi << 16);
            }
            emit(d, k0, nv);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += (uint32_t)__shfl_xor((int)sum, off);
    if (lane == 0) rowsum[row] = sum;
}

// B [K][N] int16 -> B2 [Kp][N2] int8 (N2 = round_up(2N, 16)): the bytes of B
// with every low byte ^ 0x80, zero in padding rows / columns.  One 64 x 128
// tile (rows k0.., int16 columns 128 bx..): thread t handles 8 columns
// (16 bytes) of rows (t >> 4) + 16 q, q = 0..3, and adds its columns' values
// into cs (mod 2^32).
__device__ __forceinline__ void prep_b_tile(const int16_t *__restrict__ src, int K, int N, int Kp, int N2,
                                            int8_t *__restrict__ B2, int bx, int k0, uint32_t (&cs)[8]) {
    const int tid = threadIdx.x, cg = tid & 15, rg = tid >> 4;
    const int c0 = bx * 128 + cg * 8;           // first int16 column of this thread
    const bool out_col = 2 * c0 < N2;           // this 16-byte chunk exists in B2
    uint32_t dq[4][4];
    // block-uniform: the whole 64 x 128 tile inside B with 16-byte rows
    if (((N & 7) == 0) && ((((uintptr_t)src) & 15) == 0) && bx * 128 + 128 <= N && k0 + 64 <= K) {
        // the thread's 4 rows are loaded before any is processed
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = *(const uint4 *)(src + (size_t)(k0 + rg + 16 * q) * N + c0);
            dq[q][0] = v.x, dq[q][1] = v.y, dq[q][2] = v.z, dq[q][3] = v.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = k0 + rg + 16 * q;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int16_t *p = src + (size_t)k * N + c0;
                const uint32_t lo = k < K && c0 + 2 * h < N ? (uint16_t)p[2 * h] : 0u;
                const uint32_t hi = k < K && c0 + 2 * h + 1 < N ? (uint16_t)p[2 * h + 1] : 0u;
                dq[q][h] = lo | (hi << 16);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int k = k0 + rg + 16 * q;
        if (k >= Kp) continue;
        const uint32_t(&d)[4] = dq[q];
        uint32_t o[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            cs[2 * h] += (uint32_t)(int32_t)(int16_t)(d[h] & 0xffff);
            cs[2 * h + 1] += (uint32_t)((int32_t)d[h] >> 16);
            // low byte ^ 0x80 for the valid columns only
            const uint32_t m = (k < K ? (c0 + 2 * h < N ? 0x80u : 0u) | (c0 + 2 * h + 1 < N ? 0x800000u : 0u) : 0u);
            o[h] = d[h] ^ m;
        }
        if (out_col) *(uint4 *)(B2 + (size_t)k * N2 + 2 * c0) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Column-sum partials: at most MAX_CS per column (det_kernels.h).
__host__ __device__ inline int i16_nkt(int Kp) { return (Kp + 63) / 64; }   // 64-row B tiles (Kp % 16 == 0)
__host__ __device__ inline int i16_ktp(int Kp) { return (i16_nkt(Kp) + MAX_CS - 1) / MAX_CS; }
__host__ __device__ inline int i16_ncs(int Kp) { return (i16_nkt(Kp) + i16_ktp(Kp) - 1) / i16_ktp(Kp); }

// Both operands in one launch (the two preps are independent; each alone is
// a few microseconds of fixed launch latency).  Blocks [0, na) split the A
// rows; block na + by * nbx + bx prepares the 64-row B tiles
// [by * ktp, (by + 1) * ktp) of column strip bx and writes its exact partial
// column sums to colsum[by][N] -- the GEMM epilogue adds the ncs partials,
// so no atomics and no zeroed buffer are needed.
__global__ __launch_bounds__(256) void prep_i16(const int16_t *__restrict__ A, const int16_t *__restrict__ B,
                                                int M, int N, int K, int Kp, int N2, int8_t *__restrict__ A2,
                                                int8_t *__restrict__ B2, uint32_t *__restrict__ rowsum,
                                                uint32_t *__restrict__ colsum, int na, int nbx, int ktp) {
    if ((int)blockIdx.x < na) {
        prep_a_rows(A, M, K, Kp, A2, rowsum, blockIdx.x);
        return;
    }
    __shared__ uint32_t part[16][129];
    const int t = blockIdx.x - na, bx = t % nbx, by = t / nbx;
    const int kt_end = min((by + 1) * ktp, i16_nkt(Kp));
    uint32_t cs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int kt = by * ktp; kt < kt_end; ++kt) prep_b_tile(B, K, N, Kp, N2, B2, bx, kt * 64, cs);
    const int tid = threadIdx.x, cg = tid & 15, rg = tid >> 4;
#pragma unroll
    for (int e = 0; e < 8; ++e) part[rg][cg * 8 + e] = cs[e];
    __syncthreads();
    if (tid < 128) {
        uint32_t sum = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += part[r][tid];
        const int col = bx * 128 + tid;
        if (col < N) colsum[(size_t)by * N + col] = sum;
    }
}


}  // namespace i16x

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

bool i16x_eligible(int M, int N, int K) {
    const long long Kp = ((long long)K + 15) / 16 * 16, N2 = (2LL * N + 15) / 16 * 16;
    return K >= 1 && 2LL * M * Kp < (1LL << 31) && Kp * N2 < (1LL << 31);
}

size_t i16x_workspace_bytes(int M, int N, int K) {
    const size_t Kp = ((size_t)K + 15) / 16 * 16, N2 = (2 * (size_t)N + 15) / 16 * 16;
    return align256(2 * (size_t)M * Kp) + align256(Kp * N2) + align256(4 * (size_t)M) +
           align256(4 * (size_t)i16x::i16_ncs((int)Kp) * N);
}

hipError_t launch_gemm_i16x(const int16_t *A, const int16_t *B, int32_t *C, int M, int N, int K, void *ws,
                            hipStream_t s) {
    using namespace i16x;
    const int Kp = (K + 15) / 16 * 16, N2 = (2 * N + 15) / 16 * 16;
    int8_t *A2 = (int8_t *)ws;
    int8_t *B2 = A2 + align256(2 * (size_t)M * Kp);
    uint32_t *rowsum = (uint32_t *)(B2 + align256((size_t)Kp * N2));
    uint32_t *colsum = (uint32_t *)((int8_t *)rowsum + align256(4 * (size_t)M));
    const int na = (M + 3) / 4, nbx = (N + 127) / 128, ktp = i16_ktp(Kp), ncs = i16_ncs(Kp);
    hipLaunchKernelGGL(prep_i16, dim3(na + nbx * ncs), dim3(256), 0, s, A, B, M, N, K, Kp, N2, A2, B2, rowsum,
                       colsum, na, nbx, ktp);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_gemm_i8_i16epi(A2, B2, 2 * M, N2, Kp, rowsum, colsum, ncs, C, M, N, K, s);
}

}  // namespace det
