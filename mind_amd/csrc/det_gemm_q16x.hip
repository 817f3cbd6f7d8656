// det_gemm_q16x.hip -- Q16.16 GEMM for K < 65536: limb-plane int8 MFMA for
// the bilinear part, VALU residue for the per-term floor, 12 waves per tile.
//
// Semantics (reference src/mlir/lowering.rs:9300-9410, 7074-7676, oracle
// benches/det_matmul_q16.rs:227-240):
//     C[i,j] = (int32) sum_k ( (int64)A[i,k] * (int64)B[k,j]  >>arith 16 )
// computed as C = (int32)(((S - R) mod 2^48) >> 16) with S = sum_k a b
// (from 15 limb-pair int8 MFMAs plus the bias identity) and
// R = sum_k ((lo16(a) lo16(b)) mod 2^16) (v_pk_mul_lo_u16 + v_dot2_u32_u16).
// The derivation and the limb / bias algebra are the same as the first
// generation kernel in det_gemm_limb.hip; this file changes the schedule:
//
//  * Prep (one launch for both operands): one wave per source row (A, or
//    B^T), and transposing 64x64 tiles for row-major B.  Both write the limb
//    planes [p][rows][Kp] (K-contiguous, biased bytes), the low-16 halves
//    [rows][Kp] and exact int64 row sums / column-sum partials (no atomics).
//  * Main kernel: 64x64 output tile per 768-thread workgroup, 48 KiB LDS
//    stages (limb planes + low halves of A and B for 64 k) filled by
//    direct global->LDS DMA two steps ahead (3 stages).  The waves are
//    specialised: on each SIMD one "limb wave" runs the 15 limb-pair
//    v_mfma_i32_32x32x32_i8 of a 32x32 quadrant (six shift-set
//    accumulators) and issues the DMA, and two "residue waves" compute R
//    for the whole tile, each over an eighth of each K step, with an 8x8
//    output micro-tile per lane (0.5 LDS bytes per residue term).  On
//    gfx950 an MFMA and a VALU operation of another wave on the same SIMD do
//    not execute concurrently (measured), so the kernel is bounded by MFMA
//    time plus residue VALU time per SIMD; the specialisation keeps each
//    wave's instruction stream dense and the residue LDS traffic low, and two
//    residue waves per SIMD issue VALU faster than one (a single wave waits
//    between its own instructions: 9-10% fewer cycles per tile with two).
//  * Exactness: the limb waves cover the whole K, so the shift-0 set is
//    bounded by K 2^14 and the shift-1 set by K 2^15 (exact in int32 for
//    K < 2^16); each residue wave's partial is below (K/8) 2^16 and the sum
//    of the eight below K 2^16 < 2^32.  Sets with shift >= 2 only need their
//    value mod 2^32.  The epilogue combines S, R and the bias terms in
//    uint64 and keeps bits 16..47.
#include <algorithm>

#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace q16x {

constexpr int KP_ALIGN = 64;
constexpr int BM = 64, BN = 64, BK = 64, THREADS = 768;
constexpr int PT = BM * BK;             // bytes per limb-plane tile
constexpr int LT = BM * BK * 2;         // bytes per low-16 tile
constexpr int STAGE = 8 * PT + 2 * LT;  // A and B: 4 planes + low halves
constexpr uint32_t BIAS4 = 0x80808080u;

// Byte mask of the valid elements of dword d of a 16-element run with nv
// valid elements (nv in [0, 16]).
__device__ __forceinline__ uint32_t valid_mask(int nv, int d) {
    const int r = nv - 4 * d;
    return r >= 4 ? 0xffffffffu : (r <= 0 ? 0u : (1u << (8 * r)) - 1u);
}

// 16 consecutive Q16 values (zero where invalid) -> 4 limb-plane chunks of
// 16 bytes (t_p = byte_p ^ 0x80 for p < 3, the signed top byte for p = 3,
// 0 for invalid k) and 8 dwords of packed low-16 halves.
__device__ __forceinline__ void split16(const uint32_t (&w)[16], int nv, uint4 (&pl)[4], uint4 (&lo)[2]) {
    uint32_t e[4][4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t e0, e1, e2, e3;
        transpose4x4(w[4 * d], w[4 * d + 1], w[4 * d + 2], w[4 * d + 3], e0, e1, e2, e3);
        const uint32_t x = BIAS4 & valid_mask(nv, d);
        e[0][d] = e0 ^ x;
        e[1][d] = e1 ^ x;
        e[2][d] = e2 ^ x;
        e[3][d] = e3;
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) pl[p] = make_uint4(e[p][0], e[p][1], e[p][2], e[p][3]);
    uint32_t l[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) l[h] = perm(w[2 * h + 1], w[2 * h], 0x05040100u);
    lo[0] = make_uint4(l[0], l[1], l[2], l[3]);
    lo[1] = make_uint4(l[4], l[5], l[6], l[7]);
}

// ------------------------------------------------------------------ prep
// Rows of src[R][K] (operand A, or B given as B^T): one wave per row, lane
// chunks of 16 k; rows 4 blk .. 4 blk + 3.
__device__ __forceinline__ void prep_rows(const int32_t *__restrict__ src, int R, int K, int Kp,
                                          uint8_t *__restrict__ planes, size_t plane_stride,
                                          uint16_t *__restrict__ lo16, unsigned long long *__restrict__ sums,
                                          int blk) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blk * 4 + (tid >> 6);
    if (row >= R) return;
    const int32_t *s = src + (size_t)row * K;
    const bool vec = ((K & 3) == 0) && ((((uintptr_t)src) & 15) == 0);
    long long sum = 0;
    for (int k0 = lane * 16; k0 < Kp; k0 += 1024) {
        const int nv = min(max(K - k0, 0), 16);
        uint32_t w[16];
        if (vec && nv == 16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = *(const uint4 *)(s + k0 + 4 * q);
                w[4 * q] = v.x, w[4 * q + 1] = v.y, w[4 * q + 2] = v.z, w[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) w[e] = e < nv ? (uint32_t)s[k0 + e] : 0u;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) sum += (int32_t)w[e];
        uint4 pl[4], lo[2];
        split16(w, nv, pl, lo);
        const size_t o = (size_t)row * Kp + k0;
#pragma unroll
        for (int p = 0; p < 4; ++p) *(uint4 *)(planes + p * plane_stride + o) = pl[p];
        *(uint4 *)(lo16 + o) = lo[0];
        *(uint4 *)(lo16 + o + 8) = lo[1];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane == 0) sums[row] = (unsigned long long)sum;
}

// Row-major B[K][N] -> B^T planes [p][N][Kp], low halves [N][Kp]: one
// 64 (k) x 64 (n) tile (rows k0.., columns 64 bx..); lane = 4 * column +
// k-quarter so that each column's 64 plane bytes are written by four
// neighbouring lanes.  Adds the thread's 16 values of its column into sum.
__device__ __forceinline__ void prep_cols_tile(const int32_t *__restrict__ src, int K, int N, int Kp,
                                               uint8_t *__restrict__ planes, size_t plane_stride,
                                               uint16_t *__restrict__ lo16, int32_t (*tile)[65], int bx, int k0,
                                               long long &sum) {
    const int n0 = bx * 64;
    const int tid = threadIdx.x;
    const int c = (tid & 15) * 4;
    uint4 v[4];
    if (((N & 3) == 0) && ((((uintptr_t)src) & 15) == 0) && n0 + 64 <= N && k0 + 64 <= K) {
        // block-uniform: the whole tile inside B with 16-byte rows; the four
        // loads of a thread are all in flight before any is used
#pragma unroll
        for (int pass = 0; pass < 4; ++pass)
            v[pass] = *(const uint4 *)(src + (size_t)(k0 + (tid >> 4) + 16 * pass) * N + n0 + c);
    } else {
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int k = k0 + (tid >> 4) + 16 * pass, n = n0 + c;
            const int32_t *p = src + (size_t)k * N + n;
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = k < K && n + e < N ? (uint32_t)p[e] : 0u;
            v[pass] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int kr = (tid >> 4) + 16 * pass;
        tile[kr][c + 0] = (int32_t)v[pass].x;
        tile[kr][c + 1] = (int32_t)v[pass].y;
        tile[kr][c + 2] = (int32_t)v[pass].z;
        tile[kr][c + 3] = (int32_t)v[pass].w;
    }
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6;
    const int nl = wave * 16 + (lane >> 2), kq = lane & 3;
    const int n = n0 + nl, kb = k0 + kq * 16;
    uint32_t w[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        w[e] = (uint32_t)tile[kq * 16 + e][nl];
        sum += (int32_t)w[e];
    }
    __syncthreads();   // the tile is refilled by the next call
    const int nv = min(max(K - kb, 0), 16);
    uint4 pl[4], lo[2];
    split16(w, nv, pl, lo);
    if (n < N) {
        const size_t o = (size_t)n * Kp + kb;
#pragma unroll
        for (int p = 0; p < 4; ++p) *(uint4 *)(planes + p * plane_stride + o) = pl[p];
        *(uint4 *)(lo16 + o) = lo[0];
        *(uint4 *)(lo16 + o + 8) = lo[1];
    }
}

// Column-sum partials of row-major B: at most MAX_CS per column (det_kernels.h).
__host__ __device__ inline int q16_ktp(int Kp) { return (Kp / 64 + MAX_CS - 1) / MAX_CS; }
__host__ __device__ inline int q16_ncs(int Kp) { return (Kp / 64 + q16_ktp(Kp) - 1) / q16_ktp(Kp); }

// Both operands in one launch (the two preps are independent; each alone is
// a few microseconds of fixed launch latency).  Blocks [0, na) split the A
// rows.  With B given as B^T the remaining blocks split its rows the same
// way (exact column sums, one partial).  Otherwise block na + by * nbx + bx
// prepares the 64-row tiles [by * ktp, (by + 1) * ktp) of column strip bx and
// writes its exact partial column sums to colsum[by][N]: the GEMM epilogue
// adds the partials, so no atomics and no zeroed buffer are needed.
__global__ __launch_bounds__(256) void prep_kernel(const int32_t *__restrict__ A, const int32_t *__restrict__ B,
                                                   int M, int N, int K, int Kp, uint8_t *__restrict__ Ap,
                                                   uint8_t *__restrict__ Bp, size_t a_plane, size_t b_plane,
                                                   uint16_t *__restrict__ Alo, uint16_t *__restrict__ Blo,
                                                   unsigned long long *__restrict__ rowsum,
                                                   unsigned long long *__restrict__ colsum, int na, int b_is_t,
                                                   int nbx, int ktp) {
    const int blk = blockIdx.x;
    if (blk < na) {
        prep_rows(A, M, K, Kp, Ap, a_plane, Alo, rowsum, blk);
        return;
    }
    if (b_is_t) {
        prep_rows(B, N, K, Kp, Bp, b_plane, Blo, colsum, blk - na);
        return;
    }
    __shared__ int32_t tile[64][65];
    const int t = blk - na, bx = t % nbx, by = t / nbx;
    const int kt_end = min((by + 1) * ktp, Kp / 64);
    long long sum = 0;
    for (int kt = by * ktp; kt < kt_end; ++kt) prep_cols_tile(B, K, N, Kp, Bp, b_plane, Blo, tile, bx, kt * 64, sum);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = bx * 64 + wave * 16 + (lane >> 2);
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    if ((lane & 3) == 0 && n < N) colsum[(size_t)by * N + n] = (unsigned long long)sum;
}

// ------------------------------------------------------------------ main
// Limb-plane tile [64 rows][64 k]: 16-byte chunk ch of a row is stored at
// chunk ch ^ ((row >> 2) & 3), so the 16 rows of an MFMA operand read hit 16
// distinct 16-byte bank groups.
__device__ __forceinline__ int swz_pl(int row, int ch) { return row * 64 + ((ch ^ ((row >> 2) & 3)) << 4); }
// Low-16 tile [64 rows][64 k as u16]: chunk ch (8 k) at ch ^ ((row >> 3) & 7),
// so the 8 rows 8*ly + i (ly = 0..7) read by one residue load are distinct.
__device__ __forceinline__ int swz_lo(int row, int ch) { return row * 128 + ((ch ^ ((row >> 3) & 7)) << 4); }

constexpr int NST = 3;   // LDS stages: the DMA runs two K steps ahead

// Workspace offsets (bytes) of the four operand regions, all inside one
// buffer descriptor: A planes, B^T planes, A low halves, B low halves.
struct Q16xWs {
    uint32_t a_plane, b_plane;   // bytes per limb plane (M*Kp, N*Kp)
    uint32_t bp, alo, blo;       // region offsets from the workspace base
    uint32_t bytes;              // total bytes of the four regions
};

// Residue partials in the epilogue: [4][64 lanes][RP_STRIDE] u32 (a lane's
// 8x8 block at i*8 + j; the stride makes both the dump and the MFMA-layout
// gather conflict-light).  Residue waves 4..7 write their partials, then
// waves 8..11 add theirs into the same slots (wave w+4 onto wave w).
constexpr int RP_STRIDE = 72;

// Wave roles (waves w, w+4 and w+8 share SIMD w % 4):
//  * waves 0..3 ("limb waves"): 32x32 quadrant w of the tile over the whole
//    K: the 15 limb-pair MFMAs (shift sets s = p+q in six accumulators) and
//    all of the DMA (12 loads per stage each).
//  * waves 4..11 ("residue waves"): the whole 64x64 tile over K eighth w-4
//    of every step (one 8-k chunk): an 8x8 micro-tile per lane (rows
//    8*ly+i, columns 8*lx+j), 16 LDS reads of 8 bytes per 256 VALU
//    operations.
// The residue is VALU work that no MFMA can do; giving it whole waves lets
// the SIMD issue it back to back while the limb wave's MFMAs and LDS
// traffic proceed beside it.
template <bool SPLIT>
__global__ __launch_bounds__(THREADS, 1) void q16x_kernel(
    const uint8_t *__restrict__ ws, Q16xWs L,
    const unsigned long long *__restrict__ rowsum, const unsigned long long *__restrict__ colsum, int ncs,
    int32_t *__restrict__ C, int M, int N, int Kp, int tiles_m, int tiles_n, unsigned long long kc2, int kspl_arg,
    unsigned long long *__restrict__ part) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NST * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // tile order: XCD-contiguous ids, then groups of 8 row tiles; with
    // SPLIT the kspl workgroups of a tile take consecutive ids and
    // consecutive K ranges (as even as whole 64-k steps allow, at least one
    // step each), and each writes its partial sums to part (compiled
    // separately so the unsplit kernel keeps its own code)
    const int kspl = SPLIT ? kspl_arg : 1;
    const int ntiles = tiles_m * tiles_n;
    const int pid_all = xcd_remap(blockIdx.x, ntiles * kspl);
    const int pid = pid_all / kspl, ks = pid_all - pid * kspl;
    constexpr int GM = 8;
    const int group = pid / (GM * tiles_n), first = group * GM;
    const int gsz = min(tiles_m - first, GM);
    const int inner = pid - group * GM * tiles_n;
    const int tm = first + inner % gsz, tn = inner / gsz;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kt0 = ks * (Kp / BK) / kspl, nk = (ks + 1) * (Kp / BK) / kspl - kt0;   // kspl <= Kp / BK
    uint32_t *sR = (uint32_t *)smem;   // epilogue residue partials

    if (wave < 4) {
        // ------------------------------------------------ limb waves
        const int qm = wave >> 1, qn = wave & 1;
        // DMA: a stage is 48 blocks of 1 KiB (A planes 0..15, B planes
        // 16..31, A low halves 32..39, B low halves 40..47); limb wave w
        // issues blocks 12w .. 12w+11.  Lane i of a block fills LDS slot i,
        // so it loads the global chunk that the swizzle places there.
        const v4i32 rw = rsrc_words(ws, L.bytes);
        uint32_t doff[12];
#pragma unroll
        for (int j = 0; j < 12; ++j) {
            const int b = 12 * wave + j;
            if (b < 32) {
                const int p = (b >> 2) & 3, sl = (b & 3) * 64 + lane;
                const int row = sl >> 2, ch = (sl & 3) ^ ((row >> 2) & 3);
                doff[j] = (b < 16 ? p * L.a_plane + (uint32_t)(m0 + row) * Kp
                                  : L.bp + p * L.b_plane + (uint32_t)(n0 + row) * Kp) + ch * 16;
            } else {
                const int bb = b - 32, sl = (bb & 7) * 64 + lane;
                const int row = sl >> 3, ch = (sl & 7) ^ ((row >> 3) & 7);
                doff[j] = (bb < 8 ? L.alo + 2 * (uint32_t)(m0 + row) * Kp : L.blo + 2 * (uint32_t)(n0 + row) * Kp) +
                          ch * 16;
            }
        }
        auto issue = [&](int buf, int kt) {
#pragma unroll
            for (int j = 0; j < 12; ++j) {
                const int b = 12 * wave + j;
                const uint32_t step = b < 32 ? BK : 2 * BK;
                dma16(rw, lds_addr(smem + buf * STAGE + b * 1024), (int)(doff[j] + (uint32_t)(kt0 + kt) * step));
            }
        };
        const int fr = lane & 31, fh = lane >> 5;
        v16i32 acc[6];
#pragma unroll
        for (int s = 0; s < 6; ++s)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[s][r] = 0;

        issue(0, 0);
        issue(1, nk > 1 ? 1 : 0);
        DET_WAIT_VMCNT(12);   // step 0 landed
        __builtin_amdgcn_s_barrier();
        for (int kt = 0; kt < nk; ++kt) {
            issue((kt + 2) % NST, kt + 2 < nk ? kt + 2 : nk - 1);
            __builtin_amdgcn_sched_barrier(0);
            const uint8_t *stg = smem + (kt % NST) * STAGE;
#pragma unroll
            for (int h = 0; h < 2; ++h) {   // two 32-wide K slices
                v2i64 af[4], bf[4];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    af[p] = *(const v2i64 *)(stg + p * PT + swz_pl(qm * 32 + fr, 2 * h + fh));
                    bf[p] = *(const v2i64 *)(stg + 4 * PT + p * PT + swz_pl(qn * 32 + fr, 2 * h + fh));
                }
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int p = 0; p < 4; ++p)
                        if (p + q <= 5) acc[p + q] = mfma32x32x32(af[p], bf[q], acc[p + q]);
            }
            __builtin_amdgcn_sched_barrier(0);
            DET_WAIT_VMCNT(12);   // step kt+1 (issued one iteration ago) landed
            DET_WAIT_LGKM0();
            __builtin_amdgcn_s_barrier();
        }
        DET_WAIT_VMCNT(0);     // no load past the end may still write LDS
        // this lane's column-sum partials for the epilogue: loaded now, so
        // their latency overlaps the residue waves' partial exchange
        unsigned long long cs_part[MAX_CS];
        {
            const int cc = min(n0 + qn * 32 + (lane & 31), N - 1);
#pragma unroll
            for (int i = 0; i < MAX_CS; ++i) cs_part[i] = colsum[(size_t)min(i, ncs - 1) * N + cc];
        }
        __syncthreads();       // stages free
        __syncthreads();       // residue partials of waves 4..7 written
        __syncthreads();       // waves 8..11 added theirs
        // combine in the MFMA layout: lane l, element r -> row 8(r>>2) +
        // 4(l>>5) + (r&3), column l&31 of the quadrant
        const int col_l = qn * 32 + (lane & 31);
        const int col = n0 + col_l;
        const unsigned long long c = 0x808080ull;
        // the ncs partial column sums [ncs][N] (loaded at the start)
        unsigned long long cb = 0;
#pragma unroll
        for (int i = 0; i < MAX_CS; ++i) cb += i < ncs ? cs_part[i] : 0ull;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row_l = qm * 32 + 8 * (r >> 2) + 4 * fh + (r & 3);
            const int row = m0 + row_l;
            const int ri = ((row_l >> 3) * 8 + (col_l >> 3)) * RP_STRIDE + (row_l & 7) * 8 + (col_l & 7);
            const uint32_t R = sR[ri] + sR[64 * RP_STRIDE + ri] + sR[128 * RP_STRIDE + ri] + sR[192 * RP_STRIDE + ri];
            if (row >= M || col >= N) continue;
            const long long x = (long long)acc[0][r] + ((long long)acc[1][r] << 8) - (long long)R;
            const uint32_t y = (uint32_t)acc[2][r] + ((uint32_t)acc[3][r] << 8) + ((uint32_t)acc[4][r] << 16) +
                               ((uint32_t)acc[5][r] << 24);
            const unsigned long long sr = (unsigned long long)x + ((unsigned long long)y << 16);
            if (SPLIT) {
                // this K range's (S - R) mod 2^64; the bias terms and the
                // final shift are applied once to the sum of the partials
                part[((size_t)ks * M + row) * N + col] = sr;
                continue;
            }
            const unsigned long long v = sr + c * (rowsum[row] + cb) - kc2;
            C[(size_t)row * N + col] = (int32_t)(uint32_t)(v >> 16);
        }
    } else {
        // ------------------------------------------------ residue waves
        const int kq = wave - 4;
        const int ly = lane >> 3, lx = lane & 7;
        uint32_t racc[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) racc[i][j] = 0;
        const v2u16 one = {1, 1};
        __builtin_amdgcn_s_barrier();   // step 0 landed
        for (int kt = 0; kt < nk; ++kt) {
            const uint8_t *sal = smem + (kt % NST) * STAGE + 8 * PT, *sbl = sal + LT;
            // sub-chunk sc (4 k) of this wave's eighth: chunk kq, 8-byte half sc
            uint2 av[2][8], bv[2][8];
            auto rload = [&](int sc, uint2 (&a)[8], uint2 (&b)[8]) {
                const int ch = kq, half = sc * 8;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    a[i] = *(const uint2 *)(sal + swz_lo(8 * ly + i, ch) + half);
                    b[i] = *(const uint2 *)(sbl + swz_lo(8 * lx + i, ch) + half);
                }
            };
            rload(0, av[0], bv[0]);
#pragma unroll
            for (int sc = 0; sc < 2; ++sc) {
                if (sc < 1) rload(sc + 1, av[(sc + 1) & 1], bv[(sc + 1) & 1]);
                const uint2(&a)[8] = av[sc & 1];
                const uint2(&b)[8] = bv[sc & 1];
#pragma unroll
                for (int w = 0; w < 2; ++w)
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const uint32_t x = w ? a[i].y : a[i].x;
                        uint32_t prod[8];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t y = w ? b[j].y : b[j].x;
                            prod[j] = __builtin_bit_cast(uint32_t,
                                                         __builtin_bit_cast(v2u16, x) * __builtin_bit_cast(v2u16, y));
                        }
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            racc[i][j] = __builtin_amdgcn_udot2(__builtin_bit_cast(v2u16, prod[j]), one, racc[i][j], false);
                    }
            }
            DET_WAIT_LGKM0();
            __builtin_amdgcn_s_barrier();
        }
        __syncthreads();       // stages free (matches the limb waves)
        uint32_t *dst = sR + ((kq & 3) * 64 + lane) * RP_STRIDE;
        if (kq < 4) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                *(uint4 *)(dst + i * 8) = make_uint4(racc[i][0], racc[i][1], racc[i][2], racc[i][3]);
                *(uint4 *)(dst + i * 8 + 4) = make_uint4(racc[i][4], racc[i][5], racc[i][6], racc[i][7]);
            }
        }
        __syncthreads();       // partials of waves 4..7 written
        if (kq >= 4) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint4 v = *(uint4 *)(dst + i * 8 + 4 * h);
                    v.x += racc[i][4 * h]; v.y += racc[i][4 * h + 1]; v.z += racc[i][4 * h + 2]; v.w += racc[i][4 * h + 3];
                    *(uint4 *)(dst + i * 8 + 4 * h) = v;
                }
        }
        __syncthreads();       // waves 8..11 added theirs
    }
}

// K split: C = bits 16..47 of the sum of the kspl partials (S - R over each
// K range, mod 2^64) plus the bias terms c (row sum + column sum) - K c^2:
// the same value the unsplit epilogue forms, as every term is a sum mod
// 2^64 and only bits 16..47 are kept.
__global__ __launch_bounds__(256) void split_reduce_kernel(const unsigned long long *__restrict__ part, int kspl,
                                                           const unsigned long long *__restrict__ rowsum,
                                                           const unsigned long long *__restrict__ colsum, int ncs,
                                                           int32_t *__restrict__ C, int M, int N,
                                                           unsigned long long kc2) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, mn = (size_t)M * N;
    if (i >= mn) return;
    const int row = (int)(i / (size_t)N), col = (int)(i - (size_t)row * N);
    unsigned long long v = 0, cb = 0;
    for (int k = 0; k < kspl; ++k) v += part[(size_t)k * mn + i];
    for (int k = 0; k < ncs; ++k) cb += colsum[(size_t)k * N + col];
    v += 0x808080ull * (rowsum[row] + cb) - kc2;
    C[i] = (int32_t)(uint32_t)(v >> 16);
}

}  // namespace q16x

// K splits for grids of 64 x 64 tiles that fill at most half the CUs (one
// workgroup per CU): as many as the CUs take, at most 8 and at most one per
// 64-k step, then the fewest that keep the longest split's step count.
int q16x_ksplit(int M, int N, int K, int cus) {
    const long long tiles = (long long)((M + q16x::BM - 1) / q16x::BM) * ((N + q16x::BN - 1) / q16x::BN);
    const int nk = (K + q16x::KP_ALIGN - 1) / q16x::KP_ALIGN;
    if (2 * tiles > cus || nk < 2) return 1;
    const int k = (int)std::min<long long>(std::min<long long>(8, cus / tiles), nk);
    const int steps = (nk + k - 1) / k;   // K steps of the longest split
    return (nk + steps - 1) / steps;
}

bool q16x_eligible(int M, int N, int K) {
    const long long Kp = ((long long)K + q16x::KP_ALIGN - 1) / q16x::KP_ALIGN * q16x::KP_ALIGN;
    return K >= 1 && K < 65536 && 6LL * ((long long)M + N) * Kp < (1LL << 31);
}

// Workspace layout: A planes [4][M][Kp], B^T planes [4][N][Kp], A low
// halves [M][Kp] u16, B low halves [N][Kp] u16, row sums [M] u64, column-sum
// partials [ncs][N] u64 (ncs <= MAX_CS).
size_t q16x_workspace_bytes(int M, int N, int K) {
    const size_t Kp = (size_t)((K + q16x::KP_ALIGN - 1) / q16x::KP_ALIGN) * q16x::KP_ALIGN;
    const size_t b = 6 * ((size_t)M + N) * Kp + 8 * ((size_t)M + (size_t)q16x::q16_ncs((int)Kp) * N);
    const int kspl = q16x_ksplit(M, N, K, cu_count());
    const size_t partials = kspl > 1 ? (size_t)kspl * M * N * 8 : 0;   // [kspl][M][N] u64 after the sums
    return ((b + 255) & ~(size_t)255) + partials;
}

hipError_t launch_gemm_q16x(const int32_t *A, const int32_t *B, int32_t *C, int M, int N, int K, bool b_is_t,
                            void *ws, hipStream_t s) {
    using namespace q16x;
    const int Kp = (K + KP_ALIGN - 1) / KP_ALIGN * KP_ALIGN;
    const size_t a_plane = (size_t)M * Kp, b_plane = (size_t)N * Kp;
    uint8_t *Ap = (uint8_t *)ws;
    uint8_t *Bp = Ap + 4 * a_plane;
    uint16_t *Alo = (uint16_t *)(Bp + 4 * b_plane);
    uint16_t *Blo = Alo + a_plane;
    unsigned long long *rowsum = (unsigned long long *)(Blo + b_plane);
    unsigned long long *colsum = rowsum + M;

    const int na = (M + 3) / 4, nbx = (N + 63) / 64, ktp = q16_ktp(Kp);
    const int ncs = b_is_t ? 1 : q16_ncs(Kp);
    const int nb = b_is_t ? (N + 3) / 4 : nbx * ncs;
    hipLaunchKernelGGL(prep_kernel, dim3(na + nb), dim3(256), 0, s, A, B, M, N, K, Kp, Ap, Bp, a_plane, b_plane,
                       Alo, Blo, rowsum, colsum, na, (int)b_is_t, nbx, ktp);
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const unsigned long long kc2 = (unsigned long long)K * 0x808080ull * 0x808080ull;
    Q16xWs L;
    L.a_plane = (uint32_t)a_plane;
    L.b_plane = (uint32_t)b_plane;
    L.bp = (uint32_t)(Bp - Ap);
    L.alo = (uint32_t)((uint8_t *)Alo - Ap);
    L.blo = (uint32_t)((uint8_t *)Blo - Ap);
    L.bytes = (uint32_t)((uint8_t *)(Blo + b_plane) - Ap);
    const int kspl = q16x_ksplit(M, N, K, cu_count());
    unsigned long long *part = nullptr;
    if (kspl > 1) {   // after the sums region sized for the most partials (q16x_workspace_bytes)
        const size_t b = 6 * ((size_t)M + N) * Kp + 8 * ((size_t)M + (size_t)q16_ncs(Kp) * N);
        part = (unsigned long long *)((uint8_t *)ws + ((b + 255) & ~(size_t)255));
    }
    if (kspl == 1) {
        hipLaunchKernelGGL(q16x_kernel<false>, dim3(tiles_m * tiles_n), dim3(THREADS), 0, s, Ap, L, rowsum, colsum,
                           ncs, C, M, N, Kp, tiles_m, tiles_n, kc2, 1, part);
    } else {
        hipLaunchKernelGGL(q16x_kernel<true>, dim3(tiles_m * tiles_n * kspl), dim3(THREADS), 0, s, Ap, L, rowsum,
                           colsum, ncs, C, M, N, Kp, tiles_m, tiles_n, kc2, kspl, part);
        const size_t mn = (size_t)M * N;
        hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, part, kspl, rowsum,
                           colsum, ncs, C, M, N, kc2);
    }
    return hipGetLastError();
}

}  // namespace det
