// det_gemm_limb.hip -- exact Q16.16 and int16 GEMMs on the int8 MFMA.
//
// Q16.16 (__mind_blas_matmul_mm_q16_v; reference src/mlir/lowering.rs:
// 9300-9410, 7074-7676, 9433-9805; oracle benches/det_matmul_q16.rs:227-240):
//     C[i,j] = (int32) sum_k ( (int64)A[i,k] * (int64)B[k,j]  >>arith 16 )
// int16 (build-defined GEMM whose every element is the reference int16 dot,
// benches/det_matmul_i16.rs:218-224):
//     C[i,j] = (int32) sum_k (int64)A[i,k] * (int64)B[k,j]
//
// Exactness without floating point:
//  * Limbs.  A value a (int32 / int16) is written with bytes u_0..u_{L-1},
//    the top byte signed, the others unsigned.  With t_p = u_p - 128 for the
//    unsigned bytes (the int8 reinterpretation of u_p ^ 0x80) and t_top = the
//    signed top byte:  a = T(a) + c,  T(a) = sum_p t_p 2^(8p),
//    c = 128 * sum_{p<top} 2^(8p).  Every t_p is a signed int8.
//  * Bias identity (the reference's own VNNI trick, src/mlir/gemm_tuning.rs:
//    204-214, generalised to limbs):
//        sum_k a_k b_k = sum_k T(a_k) T(b_k) + c*sum_k a_k + c*sum_k b_k - K c^2
//    and sum_k T(a)T(b) = sum_{p,q} 2^(8(p+q)) sum_k t_p(a) t_q(b): one int8
//    MFMA GEMM per limb pair, pairs of equal shift s = p+q sharing an i32
//    accumulator.
//  * Q16 per-term floor (not bilinear).  With S = sum_k a b and
//    R = sum_k ((a b) mod 2^16) = sum_k ((lo16(a) lo16(b)) mod 2^16):
//        C = (int32)( ((S - R) mod 2^48) >> 16 )
//    since each floor(p / 2^16) = (p - (p mod 2^16)) / 2^16 exactly.  Only
//    S mod 2^48 is needed, so the (3,3) pair (shift 48) is dropped: 15 limb
//    MFMAs per block.  R is computed on the VALU with v_pk_mul_lo_u16 (two
//    16-bit residues per op) and v_dot2_u32_u16 against (1,1) (adds both).
//  * Overflow.  |t_p t_q| <= 2^14.  The shift-0 set needs its exact value
//    (48 bits of S), the shift-1 set needs 40 bits: both are flushed into
//    int64 every FLUSH_K of K, far below 2^31 / (2 * 2^14).  Sets with
//    shift >= 2 only need their value mod 2^32, which the i32 MFMA
//    accumulator keeps under wrap-around.  R is flushed into uint64 at the
//    same cadence.  int16 needs only mod 2^32 for every set: no flush.
//
// Pipeline: a prep kernel splits each operand into limb planes (A as
// [plane][M][Kp], B transposed as [plane][N][Kp], Kp = K rounded up to 64,
// zero padded), the low-16 halves (Q16), and exact row / column sums; the
// main kernel is then a multi-plane int8 MFMA GEMM whose operands are all
// K-contiguous, plus the residue pass and a fused exact epilogue.
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace limb {

constexpr int KP_ALIGN = 64;

// ------------------------------------------------------------------ prep
// One 256-thread block per 64x64 tile of the source matrix src[R][Cn]
// (row-major, int32 or int16).  TRANS=false: the source row is the output
// row and the source column is k (operand A).  TRANS=true: the source row is
// k and the source column is the output row (operand B -> B^T planes).
template <typename T, int NP, bool LO16, bool TRANS>
__global__ __launch_bounds__(256) void split_kernel(const T *__restrict__ src, int R, int Cn, int K, int Kp,
                                                    int8_t *__restrict__ planes, size_t plane_stride,
                                                    uint16_t *__restrict__ lo16,
                                                    unsigned long long *__restrict__ sums) {
    __shared__ int32_t tile[64][65];
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tid = threadIdx.x;
    // coalesced load of the source tile (sign-extended to int32)
    for (int e = tid; e < 64 * 64; e += 256) {
        const int r = e >> 6, c = e & 63;
        const int gr = r0 + r, gc = c0 + c;
        tile[r][c] = (gr < R && gc < Cn) ? (int32_t)src[(size_t)gr * Cn + gc] : 0;
    }
    __syncthreads();
    // each thread: one output row, 16 consecutive k (4 groups of 4)
    const int orow_l = tid >> 2;          // 0..63
    const int kq = (tid & 3) * 16;        // 0,16,32,48
    const int orow = (TRANS ? c0 : r0) + orow_l;
    const int kbase = (TRANS ? r0 : c0) + kq;
    const int nrows = TRANS ? Cn : R;
    unsigned long long psum = 0;
    uint32_t pl[NP][4];
    uint32_t lo[8];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int p = 0; p < NP; ++p) pl[p][g] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int kl = kq + g * 4 + e;
            const int k = kbase + g * 4 + e;
            const int32_t v = TRANS ? tile[kl][orow_l] : tile[orow_l][kl];
            const bool valid = k < K;
            if (valid) psum += (unsigned long long)(long long)v;
            const uint32_t u = (uint32_t)v;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                uint32_t byte = (u >> (8 * p)) & 0xffu;
                if (p < NP - 1) byte ^= 0x80u;   // t_p = u_p - 128 as int8
                pl[p][g] |= (valid ? byte : 0u) << (8 * e);
            }
            if (LO16) {
                const uint32_t l = valid ? (u & 0xffffu) : 0u;
                if (e & 1) lo[g * 2 + (e >> 1)] |= l << 16; else lo[g * 2 + (e >> 1)] = l;
            }
        }
    }
    if (orow < nrows && kbase < Kp) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
            *(uint4 *)(planes + p * plane_stride + (size_t)orow * Kp + kbase) =
                make_uint4(pl[p][0], pl[p][1], pl[p][2], pl[p][3]);
        if (LO16) {
            uint4 *d = (uint4 *)(lo16 + (size_t)orow * Kp + kbase);
            d[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            d[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        }
    }
    // reduce the 4 threads of an output row, one atomic per row per tile
    psum += __shfl_xor(psum, 1);
    psum += __shfl_xor(psum, 2);
    if ((tid & 3) == 0 && orow < nrows) atomicAdd(sums + orow, psum);
}

__global__ void zero_u64(unsigned long long *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// ------------------------------------------------------------------ main
constexpr int BM = 64, BN = 64, BK = 64, THREADS = 256;

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}
// lo16 tile: [row][64 k] u16 = 128 bytes per row, 8 chunks of 16 bytes
__device__ __forceinline__ int swz16(int row, int chunk) {
    return row * 128 + ((chunk ^ (row & 7)) << 4);
}

template <int NP, bool Q16>
struct LimbCfg {
    static constexpr int NSHIFT = Q16 ? 6 : 2 * NP - 1;   // Q16 drops shift 6
    static constexpr int PLANE_TILE = BM * BK;            // bytes per plane tile
    static constexpr int LO_TILE = Q16 ? BM * BK * 2 : 0;
    static constexpr int STAGE = 2 * NP * PLANE_TILE + 2 * LO_TILE;
};

template <int NP, bool Q16>
__global__ __launch_bounds__(THREADS, 1) void limb_gemm_kernel(
    const int8_t *__restrict__ Ap, const int8_t *__restrict__ Bp, size_t a_plane, size_t b_plane,
    const uint16_t *__restrict__ Alo, const uint16_t *__restrict__ Blo,
    const unsigned long long *__restrict__ rowsum, const unsigned long long *__restrict__ colsum,
    int32_t *__restrict__ C, int M, int N, int K, int Kp, int tiles_m, int tiles_n, int flush_steps,
    unsigned long long bias_c) {
    using Cfg = LimbCfg<NP, Q16>;
    constexpr int NS = Cfg::NSHIFT;
    __shared__ __attribute__((aligned(16))) int8_t smem[Cfg::STAGE];
    int8_t *sA = smem;                                   // [NP][BM][64]
    int8_t *sB = smem + NP * Cfg::PLANE_TILE;            // [NP][BN][64]
    int8_t *sAlo = smem + 2 * NP * Cfg::PLANE_TILE;      // [BM][128 B]
    int8_t *sBlo = sAlo + Cfg::LO_TILE;                  // [BN][128 B]

    const int ntiles = tiles_m * tiles_n;
    const int pid = xcd_remap(blockIdx.x, ntiles);
    const int tm = pid / tiles_n, tn = pid % tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int lr = lane & 15, lg = lane >> 4;

    v4i32 acc[NS][2][2];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[s][i][j] = (v4i32){0, 0, 0, 0};
    // exact low-shift totals and residue (Q16 only)
    long long tot0[2][2][4], tot1[2][2][4];
    unsigned long long rtot[2][2][4];
    uint32_t racc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                tot0[i][j][r] = 0;
                tot1[i][j][r] = 0;
                rtot[i][j][r] = 0;
                racc[i][j][r] = 0;
            }

    const int nk = Kp / BK;
    for (int kt = 0; kt < nk; ++kt) {
        const int k0 = kt * BK;
        // ---- global -> LDS (all operands are K-contiguous, 16-byte aligned)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            // 64 rows x 4 chunks = 256 chunks per plane tile: one per thread
            const int row = tid >> 2, ch = tid & 3;
            const int ga = m0 + row, gb = n0 + row;
            uint4 va = make_uint4(0, 0, 0, 0), vb = make_uint4(0, 0, 0, 0);
            if (ga < M) va = *(const uint4 *)(Ap + p * a_plane + (size_t)ga * Kp + k0 + ch * 16);
            if (gb < N) vb = *(const uint4 *)(Bp + p * b_plane + (size_t)gb * Kp + k0 + ch * 16);
            *(uint4 *)(sA + p * Cfg::PLANE_TILE + swz(row, ch)) = va;
            *(uint4 *)(sB + p * Cfg::PLANE_TILE + swz(row, ch)) = vb;
        }
        if (Q16) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int idx = h * THREADS + tid;   // 64 rows x 8 chunks
                const int row = idx >> 3, ch = idx & 7;
                const int ga = m0 + row, gb = n0 + row;
                uint4 va = make_uint4(0, 0, 0, 0), vb = make_uint4(0, 0, 0, 0);
                if (ga < M) va = *(const uint4 *)(Alo + (size_t)ga * Kp + k0 + ch * 8);
                if (gb < N) vb = *(const uint4 *)(Blo + (size_t)gb * Kp + k0 + ch * 8);
                *(uint4 *)(sAlo + swz16(row, ch)) = va;
                *(uint4 *)(sBlo + swz16(row, ch)) = vb;
            }
        }
        __syncthreads();

        // ---- limb-pair MFMAs
        v2i64 af[NP][2], bf[NP][2];
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                af[p][i] = *(const v2i64 *)(sA + p * Cfg::PLANE_TILE + swz(wm + i * 16 + lr, lg));
                bf[p][i] = *(const v2i64 *)(sB + p * Cfg::PLANE_TILE + swz(wn + i * 16 + lr, lg));
            }
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int q = 0; q < NP; ++q) {
                if (p + q >= NS) continue;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[p + q][i][j] = mfma16x16x64(af[p][i], bf[q][j], acc[p + q][i][j]);
            }

        // ---- residue R on the VALU (Q16): lane owns rows 4*lg+r, column lr
        if (Q16) {
#pragma unroll
            for (int ch = 0; ch < 8; ++ch) {          // 8 k per chunk
                uint4 bv[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) bv[j] = *(const uint4 *)(sBlo + swz16(wn + j * 16 + lr, ch));
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint4 av = *(const uint4 *)(sAlo + swz16(wm + i * 16 + lg * 4 + r, ch));
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            uint32_t s = racc[i][j][r];
                            const v2u16 one = {1, 1};
                            s = __builtin_amdgcn_udot2(__builtin_bit_cast(v2u16, av.x) * __builtin_bit_cast(v2u16, bv[j].x), one, s, false);
                            s = __builtin_amdgcn_udot2(__builtin_bit_cast(v2u16, av.y) * __builtin_bit_cast(v2u16, bv[j].y), one, s, false);
                            s = __builtin_amdgcn_udot2(__builtin_bit_cast(v2u16, av.z) * __builtin_bit_cast(v2u16, bv[j].z), one, s, false);
                            s = __builtin_amdgcn_udot2(__builtin_bit_cast(v2u16, av.w) * __builtin_bit_cast(v2u16, bv[j].w), one, s, false);
                            racc[i][j][r] = s;
                        }
                    }
            }
        }
        __syncthreads();

        // ---- exact flush of the low shift sets (Q16)
        if (Q16 && ((kt + 1) % flush_steps == 0 || kt + 1 == nk)) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        tot0[i][j][r] += (long long)acc[0][i][j][r];
                        tot1[i][j][r] += (long long)acc[1][i][j][r];
                        rtot[i][j][r] += (unsigned long long)racc[i][j][r];
                        acc[0][i][j][r] = 0;
                        acc[1][i][j][r] = 0;
                        racc[i][j][r] = 0;
                    }
        }
    }

    // ---- epilogue
    const unsigned long long kc2 = (unsigned long long)(long long)K * bias_c * bias_c;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm + i * 16 + lg * 4 + r;
            if (row >= M) continue;
            const unsigned long long ra = rowsum[row];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = n0 + wn + j * 16 + lr;
                if (col >= N) continue;
                unsigned long long s = bias_c * (ra + colsum[col]) - kc2;
                if (Q16) {
                    s += (unsigned long long)tot0[i][j][r];
                    s += (unsigned long long)tot1[i][j][r] << 8;
                    s += (unsigned long long)(uint32_t)acc[2][i][j][r] << 16;
                    s += (unsigned long long)(uint32_t)acc[3][i][j][r] << 24;
                    s += (unsigned long long)(uint32_t)acc[4][i][j][r] << 32;
                    s += (unsigned long long)(uint32_t)acc[5][i][j][r] << 40;
                    s -= rtot[i][j][r];
                    C[(size_t)row * N + col] = (int32_t)(uint32_t)(s >> 16);
                } else {
#pragma unroll
                    for (int sh = 0; sh < NS; ++sh)
                        s += (unsigned long long)(uint32_t)acc[sh][i][j][r] << (8 * sh);
                    C[(size_t)row * N + col] = (int32_t)(uint32_t)s;
                }
            }
        }
}

}  // namespace limb

size_t limb_workspace_bytes(int M, int N, int K, int np, bool q16) {
    const size_t Kp = (size_t)((K + limb::KP_ALIGN - 1) / limb::KP_ALIGN) * limb::KP_ALIGN;
    size_t b = (size_t)np * ((size_t)M + N) * Kp;          // planes
    if (q16) b += 2 * ((size_t)M + N) * Kp;                // lo16
    b += 8 * ((size_t)M + N);                              // sums
    return (b + 255) & ~(size_t)255;
}

// B is [K][N] row-major, or (b_is_t) already transposed as [N][K].
template <typename T, int NP, bool Q16>
static hipError_t launch_limb(const T *A, const T *B, int32_t *C, int M, int N, int K, bool b_is_t, void *ws,
                              hipStream_t s) {
    using namespace limb;
    const int Kp = (K + KP_ALIGN - 1) / KP_ALIGN * KP_ALIGN;
    int8_t *base = (int8_t *)ws;
    const size_t a_plane = (size_t)M * Kp, b_plane = (size_t)N * Kp;
    int8_t *Ap = base;
    int8_t *Bp = Ap + NP * a_plane;
    uint16_t *Alo = (uint16_t *)(Bp + NP * b_plane);
    uint16_t *Blo = Q16 ? Alo + a_plane : Alo;
    unsigned long long *sums = (unsigned long long *)((int8_t *)Alo + (Q16 ? 2 * (a_plane + b_plane) : 0));
    unsigned long long *rowsum = sums, *colsum = sums + M;

    hipLaunchKernelGGL(zero_u64, dim3((M + N + 255) / 256), dim3(256), 0, s, sums, M + N);
    // A: source [M][K], tiles over (K-padded columns, rows)
    hipLaunchKernelGGL((split_kernel<T, NP, Q16, false>), dim3(Kp / 64, (M + 63) / 64), dim3(256), 0, s, A, M,
                       K, K, Kp, Ap, a_plane, Alo, rowsum);
    if (b_is_t)  // B^T source [N][K]: same split as A
        hipLaunchKernelGGL((split_kernel<T, NP, Q16, false>), dim3(Kp / 64, (N + 63) / 64), dim3(256), 0, s, B, N,
                           K, K, Kp, Bp, b_plane, Blo, colsum);
    else         // B source [K][N] -> B^T planes; tiles over (columns, K-padded rows)
        hipLaunchKernelGGL((split_kernel<T, NP, Q16, true>), dim3((N + 63) / 64, Kp / 64), dim3(256), 0, s, B, K,
                           N, K, Kp, Bp, b_plane, Blo, colsum);
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const unsigned long long bias_c = Q16 ? 0x808080ull : 0x80ull;
    // flush the exact low-shift sets every 16384 K (2 * 16384 * 2^14 = 2^29)
    const int flush_steps = 16384 / BK;
    hipLaunchKernelGGL((limb_gemm_kernel<NP, Q16>), dim3(tiles_m * tiles_n), dim3(THREADS), 0, s, Ap, Bp, a_plane,
                       b_plane, Alo, Blo, rowsum, colsum, C, M, N, K, Kp, tiles_m, tiles_n, flush_steps, bias_c);
    return hipGetLastError();
}

hipError_t launch_gemm_q16(const int32_t *A, const int32_t *B, int32_t *C, int M, int N, int K, bool b_is_t,
                           void *ws, hipStream_t s) {
    if (q16_small(M, N, K)) return launch_gemm_q16_small(A, B, C, M, N, K, b_is_t, s);
    if (q16x_eligible(M, N, K)) return launch_gemm_q16x(A, B, C, M, N, K, b_is_t, ws, s);
    return launch_limb<int32_t, 4, true>(A, B, C, M, N, K, b_is_t, ws, s);
}

size_t i16_workspace_bytes(int M, int N, int K) {
    if (i16_small(M, N, K)) return 0;
    const size_t a = limb_workspace_bytes(M, N, K, 2, false), b = i16x_workspace_bytes(M, N, K);
    return a > b ? a : b;
}

hipError_t launch_gemm_i16(const int16_t *A, const int16_t *B, int32_t *C, int M, int N, int K, void *ws,
                           hipStream_t s) {
    if (i16_small(M, N, K)) return launch_gemm_i16_small(A, B, C, M, N, K, s);
    if (i16x_eligible(M, N, K)) return launch_gemm_i16x(A, B, C, M, N, K, ws, s);
    return launch_limb<int16_t, 2, false>(A, B, C, M, N, K, false, ws, s);
}

}  // namespace det
