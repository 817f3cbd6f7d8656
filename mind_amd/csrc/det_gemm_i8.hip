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
// Kernels (routing in launch_i8_on_grid / launch_gemm_i8, all 512 threads =
// 8 waves, 2 per SIMD):
//  * gemm_i8_t256_kernel: 256 x 256 tiles of v_mfma_i32_16x16x64_i8 blocks,
//    operands moved global -> LDS by direct DMA (buffer_load ... lds), four
//    64-k stages, the two waves of a SIMD in ping-pong (one runs MFMAs while
//    the other reads LDS and issues DMA); grids that fill whole rounds of the
//    CUs (4096^3, 8192^3, the MLP layer), and the int16 limb interleave.
//  * h128::gemm_i8_h128_kernel: the same machinery on 128 x 256 tiles,
//    persistent (a tile's stores overlap the next tile's K loop), or on
//    128 x 128 tiles for grids that fit one round of them.
//  * gemm_i8_dma_kernel: 256 x 256 tiles of v_mfma_i32_32x32x32_i8 with a
//    range-checked DMA for shapes on the 16-byte grid off those multiples,
//    and the int16 epilogue on grids the t256 kernel does not take.
//  * gemm_i8_kernel: byte loads for operands off the 16-byte grid when no
//    workspace is given (otherwise pad_i8_kernel repacks them into padded
//    panels for the kernels above).
// A (K contiguous) is read from LDS with ds_read_b128 in the MFMA A layout;
// B (N contiguous) needs K-contiguous bytes per column and is read with
// gfx950's transposing ds_read_b64_tr_b8: within each 16-lane group that
// instruction returns, to lane t, byte t & 7 of the 8-byte segments
// addressed by lanes 2j + (t >> 3), j = 0..7; so when lane i addresses row
// k0 + (i >> 1), columns n0 + 8 (i & 1), lane t receives B[k0 .. k0+7][n0 + t]
// -- one column, 8 consecutive K.  Two such reads form a 16-byte B operand.
// LDS layouts are XOR-swizzled so the DMA placement and the operand reads
// are bank-conflict free.
#include <type_traits>

#include "det_common.h"
#include "det_kernels.h"

namespace det {

namespace i8g {
constexpr int BM = 256, BN = 256, BK = 64, THREADS = 512;
constexpr int TILE_BYTES = BM * BK;  // == BN * BK
constexpr int GROUP_M = 4;
constexpr int WM = 128, WN = 64;     // wave tile: 4 x 2 blocks of 32x32, 128 accumulators

// LDS has 64 four-byte banks (256 bytes per cycle).
// A tile: [256 rows][64 k]; the four 16-byte chunks of a row are XOR-swizzled
// by (row >> 2) & 3, so the 16 lanes of a ds_read_b128 (16 consecutive rows,
// one chunk) and of a ds_write_b128 (4 rows x 4 chunks) hit 16 distinct
// 16-byte bank groups.
__device__ __forceinline__ int swz_a(int row, int chunk) {
    return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}
// B tile: [64 k rows][256 n]; the sixteen 16-byte chunks of a row are
// XOR-swizzled by 2 * (row & 7).  A transposing read's 16-lane group touches
// 8 rows x one chunk: 8 distinct slots of one parity; the neighbouring group
// reads the next (opposite parity) chunk, so each pair of groups covers all
// 64 banks once.
__device__ __forceinline__ int swz_b(int row, int chunk) {
    return row * 256 + ((chunk ^ ((row & 7) << 1)) << 4);
}

typedef int v2i32 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i32 *lds_v2i32_ptr;

// Transposing read: see the header comment.  `p` is this lane's segment.
__device__ __forceinline__ v2i32 read_tr8(const int8_t *p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i32_ptr)(p));
}

// Per-thread staging of one K step: 2 x 16 bytes of A and 2 x 16 bytes of B.
struct Frag {
    uint4 a[2];
    uint4 b[2];
};

// Global -> registers.  FAST requires K % 16 == 0, N % 16 == 0, 16-byte
// aligned A and B, both below 2^31 bytes: every 16-byte chunk is then either
// fully inside or fully outside its matrix, and the outside ones are buffer
// loads at OOB_OFFSET (which return zero).
template <bool FAST>
__device__ __forceinline__ void load_tile(Frag &f, const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                          __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, int M, int N, int K,
                                          int m0, int n0, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int idx = i * THREADS + tid;
        // A: 256 rows x 4 chunks
        const int row = m0 + (idx >> 2);
        const int kc = k0 + ((idx & 3) << 4);
        // B: 64 rows x 16 chunks
        const int kr = k0 + (idx >> 4);
        const int nc = n0 + ((idx & 15) << 4);
        if (FAST) {
            f.a[i] = buf_load16(ra, row < M && kc < K ? (uint32_t)row * (uint32_t)K + (uint32_t)kc : OOB_OFFSET);
            f.b[i] = buf_load16(rb, kr < K && nc < N ? (uint32_t)kr * (uint32_t)N + (uint32_t)nc : OOB_OFFSET);
        } else {
            uint32_t w[4] = {0, 0, 0, 0}, v[4] = {0, 0, 0, 0};
            if (row < M) {
                const int8_t *p = A + (size_t)row * K;
#pragma unroll
                for (int b = 0; b < 16; ++b)
                    if (kc + b < K) w[b >> 2] |= (uint32_t)(uint8_t)p[kc + b] << ((b & 3) * 8);
            }
            if (kr < K) {
                const int8_t *p = B + (size_t)kr * N;
#pragma unroll
                for (int b = 0; b < 16; ++b)
                    if (nc + b < N) v[b >> 2] |= (uint32_t)(uint8_t)p[nc + b] << ((b & 3) * 8);
            }
            f.a[i] = make_uint4(w[0], w[1], w[2], w[3]);
            f.b[i] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
}

__device__ __forceinline__ void store_tile(const Frag &f, int8_t *sA, int8_t *sB, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int idx = i * THREADS + tid;
        *(uint4 *)(sA + swz_a(idx >> 2, idx & 3)) = f.a[i];
        *(uint4 *)(sB + swz_b(idx >> 4, idx & 15)) = f.b[i];
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
    const int wm = (wave >> 2) * WM, wn = (wave & 3) * WN;
    const int l32 = lane & 31, lh = lane >> 5;
    // transposing-read addressing of this lane (16-lane group G, index i)
    const int tg = lane >> 4, ti = lane & 15;
    const int tr_row = 16 * (tg >> 1) + (ti >> 1);   // + 32 h + 8 q
    const int tr_col = 16 * (tg & 1) + 8 * (ti & 1); // + wn + 32 j

    v16i32 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16i32){0};

    const int nk = (K + BK - 1) / BK;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, FAST ? (uint32_t)M * (uint32_t)K : 0u);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, FAST ? (uint32_t)K * (uint32_t)N : 0u);
    Frag f0, f1;
    load_tile<FAST>(f0, A, B, ra, rb, M, N, K, m0, n0, 0, tid);
    load_tile<FAST>(f1, A, B, ra, rb, M, N, K, m0, n0, BK, tid);
    store_tile(f0, smem[0][0], smem[0][1], tid);
    __syncthreads();
    load_tile<FAST>(f0, A, B, ra, rb, M, N, K, m0, n0, 2 * BK, tid);

    // Operand fragments of one K sub-step (32 k): 4 A rows-blocks, 2 B columns.
    struct Ops {
        v2i64 a[4], b[2];
    };
    auto read_ops = [&](Ops &o, const int8_t *sA, const int8_t *sB, int h) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = 32 * h + tr_row, cb = (wn + 32 * j + tr_col) >> 4, sub = tr_col & 8;
            const v2i32 lo = read_tr8(sB + swz_b(r, cb) + sub);
            const v2i32 hi = read_tr8(sB + swz_b(r + 8, cb) + sub);
            o.b[j] = __builtin_bit_cast(v2i64, (v4i32){lo.x, lo.y, hi.x, hi.y});
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) o.a[i] = *(const v2i64 *)(sA + swz_a(wm + i * 32 + l32, 2 * h + lh));
    };
    auto mma = [&](const Ops &o) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x32(o.a[i], o.b[j], acc[i][j]);
    };

    // Software pipeline, per K step kt (LDS buffer CUR holds step kt, `p0`
    // its first 32-k fragments, already read):
    //   read second-half fragments -> p1;  MFMAs on p0;
    //   stage step kt+1 (register set `next`) into the other LDS buffer;
    //   barrier (the issued MFMAs keep running through it);
    //   refill `next` with step kt+3 (two steps of lead);
    //   read the first-half fragments of step kt+1 -> p0;  MFMAs on p1.
    // Every LDS burst thus overlaps MFMAs already in flight.  The body is
    // branch-free: past the end of K the loads fall outside the matrix
    // (zeros, no memory access on the fast path), and the last stores / reads
    // touch a buffer whose contents are never used.  sched_barrier pins the
    // phase order against the scheduler.
    Ops p0, p1;
    read_ops(p0, smem[0][0], smem[0][1], 0);
#define DET_I8_STEP(CUR, next)                                                    \
    do {                                                                          \
        read_ops(p1, smem[CUR][0], smem[CUR][1], 1);                              \
        mma(p0);                                                                  \
        store_tile(next, smem[CUR ^ 1][0], smem[CUR ^ 1][1], tid);                \
        __syncthreads();                                                          \
        load_tile<FAST>(next, A, B, ra, rb, M, N, K, m0, n0, (kt + 3) * BK, tid); \
        __builtin_amdgcn_sched_barrier(0);                                        \
        read_ops(p0, smem[CUR ^ 1][0], smem[CUR ^ 1][1], 0);                      \
        mma(p1);                                                                  \
        __builtin_amdgcn_sched_barrier(0);                                        \
    } while (0)

    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        DET_I8_STEP(0, f1);
        ++kt;
        DET_I8_STEP(1, f0);
        --kt;
    }
    if (kt < nk) DET_I8_STEP(0, f1);
#undef DET_I8_STEP

    // Epilogue: lane holds C[8*(r >> 2) + 4*lh + (r & 3)][l32] of each 32x32
    // block; a store instruction covers 32 consecutive columns (128 bytes).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (row >= M) continue;
            int32_t *crow = C + (size_t)row * N;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = n0 + wn + j * 32 + l32;
                if (col < N) __builtin_nontemporal_store(acc[i][j][r], crow + col);
            }
        }
    }
}

// ---------------------------------------------------------------- DMA path
// Fast path (aligned shapes): operands go global -> LDS directly with
// buffer_load_dwordx4 ... lds (no register staging, no ds_write).  One such
// instruction writes 64 x 16 consecutive LDS bytes, lane i at offset 16 i;
// the lane -> global chunk assignment is the inverse of swz_a / swz_b, so
// the LDS tiles have exactly the layouts above.  Out-of-range chunks use
// OOB_OFFSET and land in LDS as zeros.  NSTAGE LDS stages; each wave issues
// 2 A blocks + 2 B blocks (4 instructions) per stage.
//
// Both the full-tile and the edge-tile loop use the ping-pong schedule
// described at the full-tile loop: the two waves of each SIMD alternate an
// MFMA phase and an LDS-read / DMA-issue phase, with explicit s_waitcnt
// vmcnt waits and bare s_barrier so the loads of later steps stay in flight
// across the barriers.
constexpr int NSTAGE = 4;
constexpr int DMA_PER_STAGE = 4;     // instructions per wave per stage


// Epilogues of the DMA kernel.  EPI_I8: store C.  EPI_I16: the operands are
// the int16 limb interleave built by the int16 prep (A'' row 2i / 2i+1 = low
// / high limb of A row i, B'' column 2j / 2j+1 = low / high limb of B column
// j), so each 2x2 block of the int8 product holds the four limb-pair sums of
// one int16 output; the epilogue combines them (weights 1, 2^8, 2^8, 2^16)
// and adds the bias terms, all mod 2^32.
enum { EPI_I8 = 0, EPI_I16 = 1 };
struct I16Epi {
    const uint32_t *rowsum;            // exact sums mod 2^32 of A rows
    const uint32_t *colsum;            // [ncs][N16] partial sums mod 2^32 of B columns (added here)
    int32_t *C;                        // [M16][N16] int32
    int M16, N16, ncs;
    uint32_t bias_c, kc2;              // c = 0x80 (the epilogue relies on it), K c^2 mod 2^32
};

// FULL: M % BM == 0, N % BN == 0 and K % (BK * NSTAGE) == 0 -- no bounds
// checks, and the K loop unrolled by NSTAGE so every LDS stage address is a
// compile-time offset and the DMA advances through its SGPR soffset: the
// loop issues almost no VALU besides the MFMAs (VALU and MFMA work of one
// SIMD do not overlap on gfx950).
// EPI_I8 stores C[row][col] at C + row * ldc + col for row < mst, col < nst
// (ldc = nst = N, mst = M, except for operands repacked into padded panels:
// see launch_gemm_i8); MASK = false: every row and column of the tile is
// stored (full tiles of an unpadded problem).  The int8 GEMM sends every
// full-tile shape to the h128 kernel below, so EPI_I8 runs here only on the
// edge path; the int16 GEMM (EPI_I16) uses both paths.
template <int EPI, bool FULL, bool MASK = !FULL>
__global__ __launch_bounds__(THREADS, 1) void gemm_i8_dma_kernel(const int8_t *__restrict__ A,
                                                                 const int8_t *__restrict__ B,
                                                                 int32_t *__restrict__ C, int M, int N, int K,
                                                                 int tiles_m, int tiles_n, int ldc, int mst, int nst,
                                                                 I16Epi e16) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[NSTAGE][2][TILE_BYTES];

    const int ntiles = tiles_m * tiles_n;
    const int pid = xcd_remap(blockIdx.x, ntiles);
    const int in_group = GROUP_M * tiles_n;
    const int first_m = (pid / in_group) * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int tm = first_m + (pid % in_group) % gsize;
    const int tn = (pid % in_group) / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave >> 2) * WM, wn = (wave & 3) * WN;
    const int l32 = lane & 31, lh = lane >> 5;
    // EPI_I16: this lane's column-sum partials are loaded here and held in
    // registers, so their latency hides behind the K loop (the epilogue's
    // column is known from the start: see the EPI_I16 epilogue)
    uint32_t cs_part[EPI == EPI_I16 ? MAX_CS : 1];
    if constexpr (EPI == EPI_I16) {
        const int odd = l32 & 1;
        const int cc = min(((n0 + wn) >> 1) + (l32 >> 1) + 16 * odd, e16.N16 - 1);
#pragma unroll
        for (int i = 0; i < MAX_CS; ++i) cs_part[i] = e16.colsum[(size_t)min(i, e16.ncs - 1) * e16.N16 + cc];
    }
    const int tg = lane >> 4, ti = lane & 15;
    const int tr_row = 16 * (tg >> 1) + (ti >> 1);
    const int tr_col = 16 * (tg & 1) + 8 * (ti & 1);

    const v4i32 ra = rsrc_words(A, (uint32_t)M * (uint32_t)K);
    const v4i32 rb = rsrc_words(B, (uint32_t)K * (uint32_t)N);

    // this lane's chunk of each of the wave's 2 A blocks and 2 B blocks
    uint32_t a_off[2], b_off[2];
    int a_kc[2], b_kr[2];
    bool a_ok[2], b_ok[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int slot = 64 * (2 * wave + j) + lane;
        const int ar = slot >> 2, ac = (slot & 3) ^ ((ar >> 2) & 3);
        a_ok[j] = m0 + ar < M;
        a_kc[j] = 16 * ac;
        a_off[j] = (uint32_t)(m0 + ar) * (uint32_t)K + (uint32_t)a_kc[j];
        const int br = slot >> 4, bc = (slot & 15) ^ ((br & 7) << 1);
        b_ok[j] = n0 + 16 * bc < N;
        b_kr[j] = br;
        b_off[j] = (uint32_t)br * (uint32_t)N + (uint32_t)(n0 + 16 * bc);
    }
    auto issue = [&](int stage, int k0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int blk = 2 * wave + j;
            const bool oka = a_ok[j] && k0 + a_kc[j] < K;
            dma16(ra, lds_addr(smem[stage][0] + blk * 1024), oka ? (int)(a_off[j] + (uint32_t)k0) : (int)OOB_OFFSET);
            const bool okb = b_ok[j] && k0 + b_kr[j] < K;
            dma16(rb, lds_addr(smem[stage][1] + blk * 1024),
                  okb ? (int)(b_off[j] + (uint32_t)k0 * (uint32_t)N) : (int)OOB_OFFSET);
        }
    };

    v16i32 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16i32){0};

    struct Ops {
        v2i64 a[4], b[2];
    };
    auto read_ops = [&](Ops &o, int stage, int h) {
        const int8_t *sA = smem[stage][0];
        const int8_t *sB = smem[stage][1];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = 32 * h + tr_row, cb = (wn + 32 * j + tr_col) >> 4, sub = tr_col & 8;
            const v2i32 lo = read_tr8(sB + swz_b(r, cb) + sub);
            const v2i32 hi = read_tr8(sB + swz_b(r + 8, cb) + sub);
            o.b[j] = __builtin_bit_cast(v2i64, (v4i32){lo.x, lo.y, hi.x, hi.y});
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) o.a[i] = *(const v2i64 *)(sA + swz_a(wm + i * 32 + l32, 2 * h + lh));
    };
    auto mma = [&](const Ops &o) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x32(o.a[i], o.b[j], acc[i][j]);
    };

    const int nk = (K + BK - 1) / BK;
    if constexpr (FULL) {
        // Lane offsets without k; the K step enters through soffset.  The
        // buffer unit's range check covers voffset only (soffset is added
        // after it), so a step past the end of K must not be expressed as an
        // out-of-range soffset: it re-loads the last step instead (K >= BK on
        // this path).  Those loads land in a stage whose data is never read
        // again (see the schedule below) and hit in L2.
        const uint32_t last_a = (uint32_t)(K - BK), last_b = (uint32_t)(K - BK) * (uint32_t)N;
        // LDS destinations by scalar arithmetic from one base
        const uint32_t lds_w = lds_addr(smem) + (uint32_t)(2 * wave) * 1024u;
        auto issue_f = [&](auto st_c, int k0) {
            constexpr int st = decltype(st_c)::value;
            const bool in = k0 < K;
            const uint32_t sa = in ? (uint32_t)k0 : last_a;
            const uint32_t sb = in ? (uint32_t)k0 * (uint32_t)N : last_b;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                dma16s(ra, lds_w + (uint32_t)((2 * st + 0) * TILE_BYTES + j * 1024), (int)a_off[j], sa);
                dma16s(rb, lds_w + (uint32_t)((2 * st + 1) * TILE_BYTES + j * 1024), (int)b_off[j], sb);
            }
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        using S3 = std::integral_constant<int, 3>;
        static_assert(NSTAGE == 4, "the unrolled loop below assumes 4 stages");
        // Ping-pong schedule.  Waves w and w + 4 share a SIMD; group 0
        // (waves 0-3) runs the 16 MFMAs of step j while group 1 (waves 4-7)
        // reads step j's fragments and issues its DMA share, then the groups
        // swap, so one wave's LDS / DMA phase always overlaps the other
        // wave's MFMA phase on the same SIMD (with both groups in the same
        // phase, the SIMD's MFMA pipe idled while both waited on LDS).
        // Slots between barriers:
        //   A_j = {group 0: MFMA(j),   group 1: MEM(j)}
        //   B_j = {group 0: MEM(j+1), group 1: MFMA(j)}
        // MEM(s) reads both K halves of step s (stage s % 4) and issues the
        // wave's DMA share of step s + 3 into stage (s + 3) % 4; it ends with
        // lgkmcnt(0), so every read of a stage is complete at the barrier
        // closing its slot.  Stage s % 4 is read in B_{s-1} and A_s and
        // refilled (step s + 4) in B_s and A_{s+1}: after both reads.  Before
        // the barrier closing A_j every wave waits for its own share of step
        // j + 1 (vmcnt(8): its shares of steps j + 2 and j + 3 stay in
        // flight), so the reads of step j + 1 in B_j and A_{j+1} find it in
        // LDS.  Both groups pass the same barriers (2 + 2 per step).
        issue_f(S0{}, 0);
        issue_f(S1{}, BK);
        issue_f(S2{}, 2 * BK);
        DET_WAIT_VMCNT(DMA_PER_STAGE * 2);   // step 0 landed
        __builtin_amdgcn_s_barrier();
        Ops q0, q1;
        auto mem = [&](auto st_c, int s) {
            constexpr int st = decltype(st_c)::value;
            read_ops(q0, st, 0);
            read_ops(q1, st, 1);
            issue_f(std::integral_constant<int, (st + 3) % NSTAGE>{}, (s + 3) * BK);
        };
        auto lgkm0 = [&]() { __builtin_amdgcn_s_waitcnt(0xc07f & ~(15 << 8)); };
        if (wave < 4) {
            mem(S0{}, 0);
            lgkm0();
            __builtin_amdgcn_s_barrier();
            auto step0 = [&](auto cur_c, int kt) {
                constexpr int nxt = (decltype(cur_c)::value + 1) % NSTAGE;
                __builtin_amdgcn_sched_barrier(0);
                mma(q0);
                mma(q1);
                __builtin_amdgcn_sched_barrier(0);
                DET_WAIT_VMCNT(DMA_PER_STAGE * 2);
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if (kt + 1 < nk) mem(std::integral_constant<int, nxt>{}, kt + 1);
                lgkm0();
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_barrier();
            };
            for (int kt = 0; kt < nk; kt += NSTAGE) {
                step0(S0{}, kt);
                step0(S1{}, kt + 1);
                step0(S2{}, kt + 2);
                step0(S3{}, kt + 3);
            }
        } else {
            __builtin_amdgcn_s_barrier();
            auto step1 = [&](auto cur_c, int kt) {
                __builtin_amdgcn_sched_barrier(0);
                mem(cur_c, kt);
                DET_WAIT_VMCNT(DMA_PER_STAGE * 2);
                lgkm0();
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                mma(q0);
                mma(q1);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_barrier();
            };
            for (int kt = 0; kt < nk; kt += NSTAGE) {
                step1(S0{}, kt);
                step1(S1{}, kt + 1);
                step1(S2{}, kt + 2);
                step1(S3{}, kt + 3);
            }
        }
        // the re-loads issued past the end of K must not still be writing
        // LDS when the workgroup ends
        DET_WAIT_VMCNT(0);
    } else {
    // The ping-pong schedule of the full-tile path (see there for the slot
    // structure and why every stage reuse and wait is safe), with run-time
    // stage indices, bounds-checked DMA and any number of K steps.
    static_assert(NSTAGE == 4, "the schedule below assumes 4 stages");
#pragma unroll
    for (int st = 0; st < NSTAGE - 1; ++st) issue(st, st * BK);
    DET_WAIT_VMCNT(DMA_PER_STAGE * 2);   // step 0 landed
    __builtin_amdgcn_s_barrier();
    Ops q0, q1;
    auto mem = [&](int s) {
        const int st = s % NSTAGE;
        read_ops(q0, st, 0);
        read_ops(q1, st, 1);
        issue((s + 3) % NSTAGE, (s + 3) * BK);
    };
    auto lgkm0 = [&]() { __builtin_amdgcn_s_waitcnt(0xc07f & ~(15 << 8)); };
    if (wave < 4) {
        mem(0);
        lgkm0();
        __builtin_amdgcn_s_barrier();
        for (int kt = 0; kt < nk; ++kt) {
            __builtin_amdgcn_sched_barrier(0);
            mma(q0);
            mma(q1);
            __builtin_amdgcn_sched_barrier(0);
            DET_WAIT_VMCNT(DMA_PER_STAGE * 2);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            if (kt + 1 < nk) mem(kt + 1);
            lgkm0();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
        }
    } else {
        __builtin_amdgcn_s_barrier();
        for (int kt = 0; kt < nk; ++kt) {
            __builtin_amdgcn_sched_barrier(0);
            mem(kt);
            DET_WAIT_VMCNT(DMA_PER_STAGE * 2);
            lgkm0();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            mma(q0);
            mma(q1);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
        }
    }
    // the loads issued past the end of K (re-loads of the last step on the
    // full-tile path, zero fills on the edge path) are never read; none may
    // still be writing LDS when the workgroup ends
    DET_WAIT_VMCNT(0);
    }

    if (EPI == EPI_I8) {
        // lane holds C[8*(r >> 2) + 4*lh + (r & 3)][l32] of each 32x32 block;
        // a store instruction covers 32 consecutive columns (128 bytes).
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (MASK && row >= mst) continue;
                int32_t *crow = C + (size_t)row * ldc;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = n0 + wn + j * 32 + l32;
                    // masked rows (ldc != N) store partial lines: plain stores merge them in L2
                    if constexpr (MASK) {
                        if (col < nst) crow[col] = acc[i][j][r];
                    } else {
                        __builtin_nontemporal_store(acc[i][j][r], crow + col);
                    }
                }
            }
        }
    } else {
        // Elements 2p, 2p+1 of a lane are rows 2i', 2i'+1 (low / high A limb)
        // of one column; lanes l, l^1 hold columns 2j', 2j'+1 (low / high B
        // limb).  The even lane forms c00 + 2^8 c10, the odd lane
        // 2^8 c01 + 2^16 c11, for each of the wave's two 32-column blocks
        // j = 0, 1.  One lane exchange (a DPP quad permute) per row pair
        // completes block 0's output on the even lane (it keeps its block-0
        // part and receives the odd lane's) and block 1's on the odd lane:
        // even lane 2c holds int16 column c, odd lane 2c+1 column c + 16, of
        // the same row, so every store instruction writes 2 rows x 32
        // consecutive int32 (two whole 128-byte lines).  The lanes add the
        // bias terms and store straight from registers: no LDS staging, no
        // barrier, no divergent branch when the wave's 64 x 32 output block
        // is inside C.
        const uint32_t odd = l32 & 1, oddm = 0u - odd;   // oddm: all ones on odd lanes
        const int m16_0 = (m0 + wm) >> 1, n16_0 = (n0 + wn) >> 1;
        // pair p of block row i is int16 row m16_0 + 16 i + 4 (p >> 1) + 2 lh + (p & 1)
        const int row_l = m16_0 + 2 * lh;
        const int col = n16_0 + (l32 >> 1) + 16 * (int)odd;
        // bias terms c (rowsum + colsum) - K c^2 with c = 0x80 (the limb
        // scheme's constant): rs = (rowsum << 7) - K c^2 + (colsum << 7)
        // the ncs column-sum partials (loaded at the start: clamped index,
        // masked add)
        uint32_t cs = 0;
#pragma unroll
        for (int i = 0; i < MAX_CS; ++i) cs += i < e16.ncs ? cs_part[i] : 0u;
        cs <<= 7;
        uint32_t rs[4][8];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int p = 0; p < 8; ++p)
                rs[i][p] = (e16.rowsum[min(row_l + 16 * i + 4 * (p >> 1) + (p & 1), e16.M16 - 1)] << 7) - e16.kc2 + cs;
        auto epilogue = [&](auto checked_c) {
            constexpr bool checked = decltype(checked_c)::value;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    uint32_t part[2];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t lo = (uint32_t)acc[i][j][2 * p], hi = (uint32_t)acc[i][j][2 * p + 1];
                        part[j] = (lo + (hi << 8)) << (8 * odd);   // odd lane: 2^8 c01 + 2^16 c11
                    }
                    const uint32_t send = (part[0] & oddm) | (part[1] & ~oddm);
                    const uint32_t keep = (part[1] & oddm) | (part[0] & ~oddm);
                    // lanes 2c <-> 2c+1: quad_perm [1, 0, 3, 2]
                    const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, false);
                    const int row = row_l + 16 * i + 4 * (p >> 1) + (p & 1);
                    const uint32_t o = keep + recv + rs[i][p];
                    int32_t *dst = e16.C + (size_t)row * e16.N16 + col;
                    if (!checked || (row < e16.M16 && col < e16.N16)) __builtin_nontemporal_store((int32_t)o, dst);
                }
        };
        // wave-uniform: is the wave's 64 x 32 output block inside C?
        if (m16_0 + 64 <= e16.M16 && n16_0 + 32 <= e16.N16) epilogue(std::false_type{});
        else epilogue(std::true_type{});
    }
}
// ------------------------------------------------------- 128-row tiles
// The same ping-pong schedule on a 128 x TN C tile (TN = 256 or 128), for
// grids that 256 x 256 tiles would fill poorly: small grids (2048^3: 64
// tiles of 256^2) use up to four times as many CUs, and grids whose 256 x 256
// tiles fill their last round to less than 7/8 (6144^3) balance better on
// persistent 128 x 256 tiles.  The price is a smaller wave tile (64 x 64 or
// 64 x 32): more LDS and DMA bytes per MFMA, so grids that fill whole rounds
// of 256 x 256 tiles go to the t256 kernel.
// A stage holds K = 128 as two 64-wide sub-stages, each laid out like a
// stage of the 256 x 256 kernel (A [128][64] with swz_a, B [64][TN]), so a
// barrier slot carries 16 (TN = 256) or 8 (TN = 128) MFMAs per wave; 3
// stages (144 or 96 KiB) with the DMA two steps ahead.  Full shapes only:
// M % 128 == 0, N % TN == 0, K % 128 == 0, K > 0, operands below 2^31
// bytes, aligned.  C: row stride ldc, rows below mst and columns below nst
// stored.
//
// Persistent: a workgroup walks tiles blockIdx.x, blockIdx.x + gridDim.x, ...
// (gridDim.x a multiple of 8, so every tile of a workgroup stays on its XCD).
// A finished tile's accumulators move to a second register set and its
// stores are spread over the first HEAD K steps of the next tile, after each
// step's DMA; only the last tile's stores are left exposed at the end.
namespace h128 {
// MI: 16-row MFMA blocks per wave (v_mfma_i32_16x16x64_i8; see the tile
// comment below for why not 32x32x32)
constexpr int BM = 128, WM = 64, MI = WM / 16, SUB = 2, NST = 3, KS = BK * SUB;
// Tiles are taken in groups of group_m row tiles (a launch argument): 8 for
// persistent 128 x 256 tiles (1024 rows, as the 256-row kernel's groups of
// 4), 4 for one-round 128 x 128 grids, where 2048^3 runs 4% faster with the
// smaller group (an XCD's 32 tiles then span 4 row and 8 column tiles)
inline int group_m(bool one_round_128) { return one_round_128 ? 4 : 8; }
constexpr int A_BYTES = BM * BK;
constexpr int HEAD = 6;   // K steps that carry the previous tile's stores
static_assert(HEAD % NST == 0 && HEAD >= NST, "the head must end on a stage-0 step");

// Tile width TN = 256 (waves 64 x 64: 4 x 4 blocks of 16 x 16) or 128
// (waves 64 x 32: 4 x 2 blocks, for grids that 128 x 256 tiles would leave
// half empty).  The blocks are v_mfma_i32_16x16x64_i8, not 32x32x32: the same
// LDS operand bytes and accumulator registers per wave, but on random int8
// data the 16x16x64 instruction sustains about 25% more MACs per second under
// the power-limited clock (register-only probes: 3.9 against 3.1 POP/s), as
// each MAC reads and writes half the accumulator bits.
// B sub-stage [64 k][TN n]: a transposing read's 16-lane group covers 8 rows
// of one 16-byte chunk, and the groups of k slices 0 and 1 (rows 16 apart)
// are served together, so the chunk of row r is XOR-swizzled by
// 2 (r & 7) ^ ((r >> 4) & 1) (TN = 256) or, with two 128-byte rows per
// 64-bank cycle, 2 ((r >> 1) & 3) ^ ((r >> 4) & 1) (TN = 128): the 32 lanes
// of the two groups then hit 64 distinct banks.
// A sub-stage [128 rows][64 k]: the 16-byte chunk c of row r sits at
// c ^ ((r >> 1) & 3).  A 16x16x64 operand read (lane l: row l & 15 of the
// block, chunk l >> 4) is then conflict-free; the 256-row kernel's
// (r >> 2) & 3 serves its 32-row reads but halves the rate of these
// (measured: 218 against 128 bytes per clock per CU).
__device__ __forceinline__ int swz_a16(int row, int chunk) {
    return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

template <int TN>
struct Tile {
    static constexpr int WNT = TN / 4, NJ = WNT / 16;   // 16-column blocks per wave
    static constexpr int NJD = TN / 128;                 // 1 KiB B DMA blocks per wave per sub-stage
    static constexpr int B_BYTES = BK * TN, SS = A_BYTES + B_BYTES, ST = SUB * SS;
    static constexpr int DPS = SUB * (1 + NJD);   // DMA instructions per wave per stage
    static constexpr int NSTORE = MI * NJ * 4;    // store instructions per wave per tile
    static constexpr int SPS = (NSTORE + HEAD - 1) / HEAD;   // stores per head step
    static_assert(DPS + SPS < 64, "vmcnt holds at most 63");
    static __device__ __forceinline__ int cx(int row) {
        if constexpr (TN == 256) return ((row & 7) << 1) ^ ((row >> 4) & 1);
        else return (((row >> 1) & 3) << 1) ^ ((row >> 4) & 1);
    }
    static __device__ __forceinline__ int swz(int row, int chunk) { return row * TN + ((chunk ^ cx(row)) << 4); }
    // LDS slot (16-byte unit) of a B sub-stage -> the k-row and n-chunk it holds
    static __device__ __forceinline__ void b_chunk(int slot, int &br, int &bc) {
        br = slot / (TN / 16);
        bc = (slot % (TN / 16)) ^ cx(br);
    }
    // stores carried by head step c (none outside the head)
    static __host__ __device__ constexpr int chunk_size(int c) {
        return (c < 0 || c >= HEAD) ? 0 : (NSTORE - c * SPS < SPS ? NSTORE - c * SPS : SPS);
    }
};

// f(integral_constant<int, I>) for I = I0 .. N-1, in order
template <int I, int N>
struct unroll_ic {
    template <class F>
    __device__ __forceinline__ static void run(F &&f) {
        if constexpr (I < N) {
            f(std::integral_constant<int, I>{});
            unroll_ic<I + 1, N>::run(f);
        }
    }
};

// MULTI: tiles may outnumber the workgroups (several rounds); otherwise each
// workgroup computes exactly one tile and stores it at the end.
template <bool MASK, bool MULTI, int TN>
__global__ __launch_bounds__(THREADS, 1) void gemm_i8_h128_kernel(const int8_t *__restrict__ A,
                                                                  const int8_t *__restrict__ B,
                                                                  int32_t *__restrict__ C, int M, int N, int K,
                                                                  int tiles_m, int tiles_n, int ldc, int mst,
                                                                  int nst, int group_m) {
    using T = Tile<TN>;
    constexpr int NJ = T::NJ, SS = T::SS, ST = T::ST, DPS = T::DPS, NSTORE = T::NSTORE, SPS = T::SPS;
    __shared__ __attribute__((aligned(1024))) int8_t smem[NST * ST];

    const int ntiles = tiles_m * tiles_n;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave >> 2) * WM, wn = (wave & 3) * T::WNT;
    // 16x16x64 operand lanes: row / column l16 of a block, K slice tg (16 k)
    const int l16 = lane & 15, tg = lane >> 4;

    const v4i32 ra = rsrc_words(A, (uint32_t)M * (uint32_t)K);
    const v4i32 rb = rsrc_words(B, (uint32_t)K * (uint32_t)N);
    // this lane's chunk of the wave's A block (1 KiB = 16 rows) and of its NJ
    // B blocks (1 KiB = 1024 / TN k-rows each) of a sub-stage, relative to the
    // tile origin: the inverse swizzles
    uint32_t a_rel, b_rel[T::NJD];
    {
        const int slot = 64 * wave + lane;
        const int ar = slot >> 2, ac = (slot & 3) ^ ((ar >> 1) & 3);
        a_rel = (uint32_t)ar * (uint32_t)K + (uint32_t)(16 * ac);
    }
#pragma unroll
    for (int j = 0; j < T::NJD; ++j) {
        int br, bc;
        T::b_chunk(64 * (T::NJD * wave + j) + lane, br, bc);
        b_rel[j] = (uint32_t)br * (uint32_t)N + (uint32_t)(16 * bc);
    }

    v4i32 acc[MI][NJ], prv[MI][NJ];
    int pm0 = 0, pn0 = 0;   // origin of the tile held in prv
    bool have_prev = false;

    // store e of tile (tm0, tn0) from v, e = ((i * 4 + r) * NJ / 2 + jp) * 2 + h:
    // blocks 2 jp and 2 jp + 1 of row block i hold, in element r, rows
    // 4 tg + r and columns 32 jp + l16 (+ 16).  v_permlane16_swap exchanges
    // the odd 16-lane rows of the first with the even ones of the second, so
    // each store writes two rows (h: 4 apart; lanes 0-31 and 32-63 rows 8
    // apart) of 32 consecutive columns: whole 128-byte lines.  The address is
    // a wave-uniform row pointer plus this lane's byte offset (8 (lane >> 5)
    // rows and lane & 31 columns, below 2^32 since ldc < 2^24)
    static_assert(NJ % 2 == 0, "column blocks are stored in pairs");
    const int l32 = lane & 31, lh = lane >> 5;
    const uint32_t lane_b = (uint32_t)(8 * lh) * (uint32_t)ldc * 4u + (uint32_t)l32 * 4u;
    // Non-temporal stores (streamed past L2) for whole rows; a masked tile
    // stores rows of ldc != N words, whose partial 128-byte lines merge
    // better in L2 (4095^3: 3% faster with plain stores, 4096^3 slower)
    auto store_c = [&](const v4i32 (&v)[MI][NJ], int tm0, int tn0, int e) __attribute__((always_inline)) {
        const int h = e & 1, jp = (e >> 1) % (NJ / 2), r = (e / NJ) & 3, i = e / (4 * NJ);
        const auto sw = __builtin_amdgcn_permlane16_swap((unsigned)v[i][2 * jp][r], (unsigned)v[i][2 * jp + 1][r],
                                                         false, false);
        const int32_t val = (int32_t)(h ? sw[1] : sw[0]);
        const int rowu = tm0 + wm + i * 16 + r + 4 * h;   // wave-uniform part
        const int colu = tn0 + wn + 32 * jp;
        int32_t *dst = (int32_t *)((char *)(C + (size_t)rowu * ldc + colu) + lane_b);
        if constexpr (MASK) {
            if (rowu + 8 * lh < mst && colu + l32 < nst) *dst = val;
        } else {
            __builtin_nontemporal_store(val, dst);
        }
    };
    auto store_prev = [&](int e) __attribute__((always_inline)) { store_c(prv, pm0, pn0, e); };

    const int nk = K / KS;
    // K advances through soffset, which the range check does not cover: a
    // step past the end re-loads the last step (into a stage never read again)
    const uint32_t last_a = (uint32_t)(K - KS), last_b = (uint32_t)(K - KS) * (uint32_t)N;
    const uint32_t base = lds_addr(smem);

    for (int t = blockIdx.x; t < ntiles; t += MULTI ? gridDim.x : ntiles) {
        const int pid = xcd_remap(t, ntiles);
        const int in_group = group_m * tiles_n;
        const int first_m = (pid / in_group) * group_m;
        const int gsize = min(tiles_m - first_m, group_m);
        const int tm = first_m + (pid % in_group) % gsize;
        const int tn = (pid % in_group) / gsize;
        const int m0 = tm * BM, n0 = tn * TN;
        const uint32_t a_off = (uint32_t)m0 * (uint32_t)K + a_rel;
        uint32_t b_off[T::NJD];
#pragma unroll
        for (int j = 0; j < T::NJD; ++j) b_off[j] = b_rel[j] + (uint32_t)n0;

#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[i][j] = (v4i32){0, 0, 0, 0};

        // the operands of one 64-k sub-stage: lane (l16, tg) holds k
        // 16 tg .. 16 tg + 15 of A row l16 / B column l16 of each block
        struct Ops {
            v2i64 a[MI], b[NJ];
        };
        auto read_ops = [&](Ops &o, int stage, int sub) __attribute__((always_inline)) {
            const int8_t *sA = smem + stage * ST + sub * SS;
            const int8_t *sB = sA + A_BYTES;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                // transposing reads: lane l16 of the group gets column
                // wn + 16 j + l16, rows 16 tg .. +7 (lo) and +8 .. +15 (hi)
                const int r = 16 * tg + (l16 >> 1), cb = (wn + 16 * j) >> 4, sub8 = 8 * (l16 & 1);
                const v2i32 lo = read_tr8(sB + T::swz(r, cb) + sub8);
                const v2i32 hi = read_tr8(sB + T::swz(r + 8, cb) + sub8);
                o.b[j] = __builtin_bit_cast(v2i64, (v4i32){lo.x, lo.y, hi.x, hi.y});
            }
#pragma unroll
            for (int i = 0; i < MI; ++i) o.a[i] = *(const v2i64 *)(sA + swz_a16(wm + i * 16 + l16, tg));
        };
        // DMA instruction d (0 .. DPS-1) of this wave's share of the K step at
        // byte offset k0 into stage st: sub-stage d / (1 + NJD), then its A
        // block or one of its B blocks
        auto dma_one = [&](auto st_c, auto d_c, int k0) __attribute__((always_inline)) {
            constexpr int st = decltype(st_c)::value, d = decltype(d_c)::value;
            constexpr int u = d / (1 + T::NJD), r = d % (1 + T::NJD);
            const bool in = k0 < K;
            if constexpr (r == 0) {
                const uint32_t sa = in ? (uint32_t)k0 : last_a;
                dma16s(ra, base + (uint32_t)(st * ST + u * SS) + (uint32_t)wave * 1024u, (int)a_off,
                       sa + (uint32_t)(u * BK));
            } else {
                const uint32_t sb = in ? (uint32_t)k0 * (uint32_t)N : last_b;
                dma16s(rb, base + (uint32_t)(st * ST + u * SS + A_BYTES) + (uint32_t)(T::NJD * wave + r - 1) * 1024u,
                       (int)b_off[r - 1], sb + (uint32_t)(u * BK) * (uint32_t)N);
            }
        };
        auto issue_f = [&](auto st_c, int k0) __attribute__((always_inline)) {
            unroll_ic<0, DPS>::run([&](auto d_c) __attribute__((always_inline)) { dma_one(st_c, d_c, k0); });
        };
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        static_assert(NST == 3, "the unrolled loop below assumes 3 stages");
        // Ping-pong schedule as in gemm_i8_dma_kernel: slots A_j = {group 0:
        // MFMA(j), group 1: MEM(j)}, B_j = {group 0: MEM(j+1), group 1: MFMA(j)}.
        // MEM(s) reads step s (stage s % 3) into registers.  The DMA refills
        // can be split between the phases (DH instructions per step in MEM);
        // with the 16x16x64 blocks all of them go into the MFMA phase, one
        // after every GAP MFMAs (DH = 1, 2 or 3 measured equal or slower):
        //   MEM(s): the first DH instructions of step s + 2, into (s + 2) % 3
        //   group 0, MFMA(j) in A_j: the rest of step j + 2
        //   group 1, MFMA(j) in B_j: the rest of step j + 3, into j % 3
        // Step s - 1 (stage (s + 2) % 3) was read in B_{s-2} and A_{s-1}, step
        // j in B_{j-1} and A_j: both before their refills.  Before the barrier
        // closing A_j each wave waits for its share of step j + 1 (read from
        // B_j on) with vmcnt(DPS + the stores of its last MEM phase): vector
        // memory operations complete in issue order, and only that many were
        // issued after it (for group 1 also the stores of the MEM phase
        // before, which this waits for as well).
        // All LDS reads of the previous tile ended before its last barrier,
        // and its past-the-end re-loads landed (vmcnt(0) below), so the
        // prologue refills stages at once: steps 0 and 1, and for group 1 the
        // second half of step 2 (its MFMA phases refill three steps ahead).
        constexpr int DH = 0;
        issue_f(S0{}, 0);
        issue_f(S1{}, KS);
        if (wave >= 4) {
            unroll_ic<DH, DPS>::run([&](auto d_c) __attribute__((always_inline)) { dma_one(S2{}, d_c, 2 * KS); });
            DET_WAIT_VMCNT(DPS + DPS - DH);   // step 0 landed
        } else {
            DET_WAIT_VMCNT(DPS);
        }
        __builtin_amdgcn_s_barrier();
        Ops q0, q1;
        // MEM(s) from stage ST, carrying head chunk CH of the previous tile's stores
        auto mem = [&](auto st_c, auto ch_c, int s) __attribute__((always_inline)) {
            constexpr int st = decltype(st_c)::value, ch = decltype(ch_c)::value;
            read_ops(q0, st, 0);
            read_ops(q1, st, 1);
            unroll_ic<0, DH>::run([&](auto d_c) __attribute__((always_inline)) {
                dma_one(std::integral_constant<int, (st + 2) % NST>{}, d_c, (s + 2) * KS);
            });
            if constexpr (T::chunk_size(ch) > 0) {
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (MASK) {
                    // the masked stores' row / column tests, hoisted out of
                    // the K loop for all NSTORE stores, spill the LDS read
                    // addresses (reloaded with vmcnt(0) waits that drain the
                    // DMA): an opaque copy of the tile origin keeps them here
                    int pm = pm0, pn = pn0;
                    asm volatile("" : "+s"(pm), "+s"(pn));
#pragma unroll
                    for (int e = ch * SPS; e < ch * SPS + T::chunk_size(ch); ++e) store_c(prv, pm, pn, e);
                } else {
#pragma unroll
                    for (int e = ch * SPS; e < ch * SPS + T::chunk_size(ch); ++e) store_prev(e);
                }
            }
        };
        // the MFMA phase: MFMA e = (sub-stage, i, j) in the order (q0, q1);
        // DMA instructions DH .. DPS-1 of the refill of stage SD with the step
        // at k0 spread over it, one after every GAP MFMAs
        auto mma_dma = [&](auto sd_c, int k0) __attribute__((always_inline)) {
            constexpr int NM = 2 * MI * NJ, GAP = DPS > DH ? NM / (DPS - DH) : NM;
            unroll_ic<0, NM>::run([&](auto e_c) __attribute__((always_inline)) {
                constexpr int e = decltype(e_c)::value, q = e / (MI * NJ), i = (e / NJ) % MI, j = e % NJ;
                const Ops &o = q == 0 ? q0 : q1;
                acc[i][j] = mfma16x16x64(o.a[i], o.b[j], acc[i][j]);
                if constexpr (e % GAP == 0 && DH + e / GAP < DPS) {
                    __builtin_amdgcn_sched_barrier(0);
                    dma_one(sd_c, std::integral_constant<int, DH + e / GAP>{}, k0);
                    __builtin_amdgcn_sched_barrier(0);
                }
            });
        };
        using NONE = std::integral_constant<int, -1>;
        // a tile carries the previous one's stores in its head when it has at
        // least HEAD steps; otherwise they go out here, all at once
        const bool spread = MULTI && have_prev && nk >= HEAD;
        if (MULTI && have_prev && !spread)
#pragma unroll
            for (int e = 0; e < NSTORE; ++e) store_prev(e);
        if (wave < 4) {
            // step kt: W = head chunk issued by MEM(kt), whose stores may still
            // be in flight; MEM(kt + 1) carries chunk kt + 1
            auto step0 = [&](auto cur_c, auto w_c, int kt) __attribute__((always_inline)) {
                constexpr int cur = decltype(cur_c)::value, nxt = (cur + 1) % NST, w = decltype(w_c)::value;
                using CH = std::integral_constant<int, (w >= 0 && w + 1 < HEAD) ? w + 1 : -1>;
                __builtin_amdgcn_sched_barrier(0);
                mma_dma(std::integral_constant<int, (cur + 2) % NST>{}, (kt + 2) * KS);
                __builtin_amdgcn_sched_barrier(0);
                DET_WAIT_VMCNT(DPS + T::chunk_size(w));
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if (kt + 1 < nk) mem(std::integral_constant<int, nxt>{}, CH{}, kt + 1);
                DET_WAIT_LGKM0();
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_barrier();
            };
            int kt = 0;
            if (spread) {
                mem(S0{}, std::integral_constant<int, 0>{}, 0);
                DET_WAIT_LGKM0();
                __builtin_amdgcn_s_barrier();
                unroll_ic<0, HEAD>::run([&](auto ic) __attribute__((always_inline)) {
                    constexpr int i = decltype(ic)::value;
                    step0(std::integral_constant<int, i % NST>{}, ic, i);
                });
                kt = HEAD;
            } else {
                mem(S0{}, NONE{}, 0);
                DET_WAIT_LGKM0();
                __builtin_amdgcn_s_barrier();
            }
            for (; kt + NST <= nk; kt += NST) {
                step0(S0{}, NONE{}, kt);
                step0(S1{}, NONE{}, kt + 1);
                step0(S2{}, NONE{}, kt + 2);
            }
            if (kt < nk) step0(S0{}, NONE{}, kt);
            if (kt + 1 < nk) step0(S1{}, NONE{}, kt + 1);
        } else {
            __builtin_amdgcn_s_barrier();
            auto step1 = [&](auto cur_c, auto ch_c, int kt) __attribute__((always_inline)) {
                __builtin_amdgcn_sched_barrier(0);
                mem(cur_c, ch_c, kt);
                DET_WAIT_VMCNT(DPS + T::chunk_size(decltype(ch_c)::value));
                DET_WAIT_LGKM0();
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                mma_dma(cur_c, (kt + 3) * KS);
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_barrier();
            };
            int kt = 0;
            if (spread) {
                unroll_ic<0, HEAD>::run([&](auto ic) __attribute__((always_inline)) {
                    constexpr int i = decltype(ic)::value;
                    step1(std::integral_constant<int, i % NST>{}, ic, i);
                });
                kt = HEAD;
            }
            for (; kt + NST <= nk; kt += NST) {
                step1(S0{}, NONE{}, kt);
                step1(S1{}, NONE{}, kt + 1);
                step1(S2{}, NONE{}, kt + 2);
            }
            if (kt < nk) step1(S0{}, NONE{}, kt);
            if (kt + 1 < nk) step1(S1{}, NONE{}, kt + 1);
        }
        // the re-loads issued past the end of K must not still be writing LDS
        // when the next tile refills its first stages
        DET_WAIT_VMCNT(0);

        if constexpr (MULTI) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) prv[i][j] = acc[i][j];
            pm0 = m0;
            pn0 = n0;
            have_prev = true;
        } else {
#pragma unroll
            for (int e = 0; e < NSTORE; ++e) store_c(acc, m0, n0, e);
        }
    }
    if (MULTI && have_prev)
#pragma unroll
        for (int e = 0; e < NSTORE; ++e) store_prev(e);
}
}  // namespace h128

// 256 x 256 tiles of 16x16x64 blocks: eight waves (two per SIMD) of 128 x 64
// (8 x 4 blocks), K steps of 64 through four LDS stages of 32 KiB.  A 64-k
// step brings 32 KiB per CU into LDS by DMA for 256 x 256 x 64 MACs, two
// thirds of the h128 tiles' 48 KiB per 128 x 256 x 128; that L2-to-LDS stream
// sets the h128 step time, so on grids of at least one full round of these
// tiles the larger tile runs its K loop faster, though its stores are not
// overlapped with a next tile (the accumulators fill the registers).
namespace t256 {
constexpr int BM = 256, TN = 256, WM = 128, WN = 64, MI = WM / 16, NJ = WN / 16;
constexpr int NST = 4, A_BYTES = BM * BK, B_BYTES = BK * TN, SS = A_BYTES + B_BYTES;   // 32 KiB stages
constexpr int DPS = 4;       // DMA instructions per wave per step: 2 A and 2 B blocks of 1 KiB
constexpr int NSTORE = MI * NJ * 4;
using TB = h128::Tile<TN>;   // B stage [64 k][256 n], the h128 layout
using h128::unroll_ic;
// Row tiles per group sharing B column panels: 4 (1024 rows) for grids of
// several rounds, 2 for one round (4096^3: 57.0 against 59.1 us with 4; the
// MLP layer and 8192^3 are 1% slower with 2, and 3-5% with 1)
inline int group_m(int rounds) { return rounds == 1 ? 2 : 4; }

// EPI_I8: C[row][col] at C + row * ldc + col for row < mst, col < nst (MASK;
// all rows and columns of the tile otherwise).  EPI_I16: the int16 limb
// interleave's epilogue (see gemm_i8_dma_kernel), into e16.C.
template <bool MASK, int EPI = EPI_I8>
__global__ __launch_bounds__(THREADS, 1) void gemm_i8_t256_kernel(const int8_t *__restrict__ A,
                                                                  const int8_t *__restrict__ B,
                                                                  int32_t *__restrict__ C, int M, int N, int K,
                                                                  int tiles_m, int tiles_n, int ldc, int mst, int nst,
                                                                  int group_m, I16Epi e16) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[NST * SS];

    // tiles taken in groups of group_m row tiles that share B column panels
    const int ntiles = tiles_m * tiles_n;
    const int pid = xcd_remap(blockIdx.x, ntiles);
    const int in_group = group_m * tiles_n;
    const int first_m = (pid / in_group) * group_m;
    const int gsize = min(tiles_m - first_m, group_m);
    const int m0 = (first_m + (pid % in_group) % gsize) * BM, n0 = ((pid % in_group) / gsize) * TN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave >> 2) * WM, wn = (wave & 3) * WN;
    const int l16 = lane & 15, tg = lane >> 4;
    const int l32 = lane & 31, lh = lane >> 5;
    // EPI_I16: this lane's int16 output column is the same for all its
    // stores (see the epilogue), so its column-sum partials load here and
    // their latency hides behind the K loop
    const int col16 = ((n0 + wn) >> 1) + 16 * ((lane >> 4) & 1) + 8 * (lane & 1) + ((lane & 15) >> 1);
    uint32_t cs_part[EPI == EPI_I16 ? MAX_CS : 1];
    if constexpr (EPI == EPI_I16) {
        const int cc = min(col16, e16.N16 - 1);
#pragma unroll
        for (int i = 0; i < MAX_CS; ++i) cs_part[i] = e16.colsum[(size_t)min(i, e16.ncs - 1) * e16.N16 + cc];
    }

    const v4i32 ra = rsrc_words(A, (uint32_t)M * (uint32_t)K);
    const v4i32 rb = rsrc_words(B, (uint32_t)K * (uint32_t)N);
    // this lane's chunk of the wave's two A blocks (16 rows x 64 k) and two B
    // blocks (4 k-rows x 256 n) of a stage: the inverse swizzles
    uint32_t a_off[2], b_off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int slot = 64 * (2 * wave + j) + lane;
        const int ar = slot >> 2, ac = (slot & 3) ^ ((ar >> 1) & 3);
        a_off[j] = (uint32_t)(m0 + ar) * (uint32_t)K + (uint32_t)(16 * ac);
        int br, bc;
        TB::b_chunk(slot, br, bc);
        b_off[j] = (uint32_t)br * (uint32_t)N + (uint32_t)(n0 + 16 * bc);
    }
    // K advances through soffset, which the range check does not cover: a
    // step past the end re-loads the last step (into a stage never read again)
    const uint32_t last_a = (uint32_t)(K - BK), last_b = (uint32_t)(K - BK) * (uint32_t)N;
    const uint32_t base = lds_addr(smem);
    // DMA instruction d of this wave's share of the step at k0 into stage st
    auto dma_one = [&](auto st_c, auto d_c, int k0) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value, d = decltype(d_c)::value;
        const bool in = k0 < K;
        if constexpr (d < 2) {
            dma16s(ra, base + (uint32_t)(st * SS) + (uint32_t)(2 * wave + d) * 1024u, (int)a_off[d],
                   in ? (uint32_t)k0 : last_a);
        } else {
            dma16s(rb, base + (uint32_t)(st * SS + A_BYTES) + (uint32_t)(2 * wave + d - 2) * 1024u, (int)b_off[d - 2],
                   in ? (uint32_t)k0 * (uint32_t)N : last_b);
        }
    };
    auto issue_f = [&](auto st_c, int k0) __attribute__((always_inline)) {
        unroll_ic<0, DPS>::run([&](auto d_c) __attribute__((always_inline)) { dma_one(st_c, d_c, k0); });
    };

    v4i32 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = (v4i32){0, 0, 0, 0};

    // the operands of one step: lane (l16, tg) holds k 16 tg .. 16 tg + 15 of
    // A row l16 / B column l16 of each block
    struct Ops {
        v2i64 a[MI], b[NJ];
    } q;
    auto mem = [&](auto st_c) __attribute__((always_inline)) {
        const int8_t *sA = smem + decltype(st_c)::value * SS;
        const int8_t *sB = sA + A_BYTES;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int r = 16 * tg + (l16 >> 1), cb = (wn + 16 * j) >> 4, sub8 = 8 * (l16 & 1);
            const v2i32 lo = read_tr8(sB + TB::swz(r, cb) + sub8);
            const v2i32 hi = read_tr8(sB + TB::swz(r + 8, cb) + sub8);
            q.b[j] = __builtin_bit_cast(v2i64, (v4i32){lo.x, lo.y, hi.x, hi.y});
        }
#pragma unroll
        for (int i = 0; i < MI; ++i) q.a[i] = *(const v2i64 *)(sA + h128::swz_a16(wm + i * 16 + l16, tg));
    };
    // the MFMA phase
    auto mma = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x64(q.a[i], q.b[j], acc[i][j]);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    static_assert(NST == 4, "the unrolled loop below assumes 4 stages");
    // Ping-pong: waves w and w + 4 share a SIMD.  Slots between barriers
    //   A_j = {group 0: MFMA(j), group 1: MEM(j)}, B_j = {group 0: MEM(j+1), group 1: MFMA(j)}
    // MEM(s) reads step s from stage s % 4 and issues the wave's DMA share
    // of a later step: group 1 in A_j step j + 3 into stage (j + 3) % 4 (step
    // j - 1, read in B_{j-2} and A_{j-1}), group 0 in B_j step j + 4 into
    // stage j % 4 (step j, read in B_{j-1} and A_j).  Before the barrier
    // closing A_j each wave waits for its share of step j + 1: two of its
    // later steps (8 DMA instructions) stay in flight.  The prologue fills
    // steps 0-2, and step 3 for group 0.  (Spread over the MFMA phase
    // instead, as the h128 kernel does, the DMA measured 2% slower here.)
    const int nk = K / BK;
    issue_f(S0{}, 0);
    issue_f(S1{}, BK);
    issue_f(S2{}, 2 * BK);
    if (wave < 4) {
        issue_f(S3{}, 3 * BK);
        DET_WAIT_VMCNT(3 * DPS);
    } else {
        DET_WAIT_VMCNT(2 * DPS);
    }
    __builtin_amdgcn_s_barrier();
    if (wave < 4) {
        mem(S0{});
        DET_WAIT_LGKM0();
        __builtin_amdgcn_s_barrier();
        auto step0 = [&](auto cur_c, int kt) __attribute__((always_inline)) {
            constexpr int cur = decltype(cur_c)::value;
            __builtin_amdgcn_sched_barrier(0);
            mma();
            __builtin_amdgcn_sched_barrier(0);
            DET_WAIT_VMCNT(2 * DPS);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            mem(std::integral_constant<int, (cur + 1) % NST>{});   // past the last step: unused reads
            issue_f(std::integral_constant<int, cur>{}, (kt + 4) * BK);
            DET_WAIT_LGKM0();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
        };
        for (int kt = 0; kt < nk; kt += NST) {
            step0(S0{}, kt);
            step0(S1{}, kt + 1);
            step0(S2{}, kt + 2);
            step0(S3{}, kt + 3);
        }
    } else {
        __builtin_amdgcn_s_barrier();
        auto step1 = [&](auto cur_c, int kt) __attribute__((always_inline)) {
            __builtin_amdgcn_sched_barrier(0);
            mem(cur_c);
            issue_f(std::integral_constant<int, (decltype(cur_c)::value + 3) % NST>{}, (kt + 3) * BK);
            DET_WAIT_VMCNT(2 * DPS);
            DET_WAIT_LGKM0();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            mma();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
        };
        for (int kt = 0; kt < nk; kt += NST) {
            step1(S0{}, kt);
            step1(S1{}, kt + 1);
            step1(S2{}, kt + 2);
            step1(S3{}, kt + 3);
        }
    }
    // the re-loads issued past the end of K must not outlive the workgroup
    DET_WAIT_VMCNT(0);

    if constexpr (EPI == EPI_I16) {
        // Lane l, element r of block (i, j) holds int8-product row 16 i + 4 tg
        // + r (int16 row 8 i + 2 tg + (r >> 1), A limb r & 1) and column
        // 16 j + l16 (int16 column 8 j + (l16 >> 1), B limb l16 & 1).  Per
        // row pair p = r >> 1 a lane forms c_0Y + 2^8 c_1Y, shifted by 8 on
        // odd lanes (B limb 1); one DPP exchange between lanes 2c and 2c + 1
        // completes block 2 jp on the even lane and block 2 jp + 1 on the odd
        // one (int16 columns 16 jp + c and 16 jp + 8 + c), and
        // v_permlane16_swap of the jp = 0 and 1 results joins lane groups
        // (tg 0, 1) and (2, 3): every store then writes two int16 rows (8 i +
        // 2 s + p and 4 below) of 32 consecutive int32 (whole 128-byte lines),
        // lane l at column col16.
        const uint32_t odd = lane & 1, oddm = 0u - odd;
        const int m16_0 = (m0 + wm) >> 1, n16_0 = (n0 + wn) >> 1;   // the wave's 64 x 32 output block
        uint32_t cs = 0;
#pragma unroll
        for (int i = 0; i < MAX_CS; ++i) cs += i < e16.ncs ? cs_part[i] : 0u;
        // bias terms c (rowsum + colsum) - K c^2, c = 0x80
        cs = (cs << 7) - e16.kc2;
        auto epilogue = [&](auto checked_c) __attribute__((always_inline)) {
            constexpr bool checked = decltype(checked_c)::value;
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    uint32_t v[2];
#pragma unroll
                    for (int jp = 0; jp < 2; ++jp) {
                        uint32_t part[2];
#pragma unroll
                        for (int jj = 0; jj < 2; ++jj) {
                            const uint32_t lo = (uint32_t)acc[i][2 * jp + jj][2 * p];
                            const uint32_t hi = (uint32_t)acc[i][2 * jp + jj][2 * p + 1];
                            part[jj] = (lo + (hi << 8)) << (8 * odd);
                        }
                        const uint32_t send = (part[0] & oddm) | (part[1] & ~oddm);
                        const uint32_t keep = (part[1] & oddm) | (part[0] & ~oddm);
                        // lanes 2c <-> 2c+1: quad_perm [1, 0, 3, 2]
                        v[jp] = keep + (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0xB1, 0xF, 0xF, false);
                    }
                    const auto sw = __builtin_amdgcn_permlane16_swap(v[0], v[1], false, false);
#pragma unroll
                    for (int sidx = 0; sidx < 2; ++sidx) {
                        const int row = m16_0 + 8 * i + 2 * sidx + p + 4 * lh;
                        const uint32_t o = (uint32_t)sw[sidx] + (e16.rowsum[min(row, e16.M16 - 1)] << 7) + cs;
                        int32_t *dst = e16.C + (size_t)row * e16.N16 + col16;
                        if (!checked || (row < e16.M16 && col16 < e16.N16)) __builtin_nontemporal_store((int32_t)o, dst);
                    }
                }
        };
        // wave-uniform: is the wave's 64 x 32 output block inside C?
        if (m16_0 + 64 <= e16.M16 && n16_0 + 32 <= e16.N16) epilogue(std::false_type{});
        else epilogue(std::true_type{});
        return;
    }
    // stores as in the h128 kernel: blocks 2 jp and 2 jp + 1 of row block i
    // paired by v_permlane16_swap, two rows (h: 4 apart; lane halves 8 apart)
    // of 32 consecutive columns (one 128-byte line) per instruction
    const uint32_t lane_b = (uint32_t)(8 * lh) * (uint32_t)ldc * 4u + (uint32_t)l32 * 4u;
#pragma unroll
    for (int e = 0; e < NSTORE; ++e) {
        const int h = e & 1, jp = (e >> 1) % (NJ / 2), r = (e / NJ) & 3, i = e / (4 * NJ);
        const auto sw = __builtin_amdgcn_permlane16_swap((unsigned)acc[i][2 * jp][r], (unsigned)acc[i][2 * jp + 1][r],
                                                         false, false);
        const int32_t val = (int32_t)(h ? sw[1] : sw[0]);
        const int rowu = m0 + wm + i * 16 + r + 4 * h;
        const int colu = n0 + wn + 32 * jp;
        int32_t *dst = (int32_t *)((char *)(C + (size_t)rowu * ldc + colu) + lane_b);
        if constexpr (MASK) {
            if (rowu + 8 * lh < mst && colu + l32 < nst) *dst = val;
        } else {
            __builtin_nontemporal_store(val, dst);
        }
    }
}
}  // namespace t256
}  // namespace i8g

// Compute units of the current device (cached per device).
int cu_count() {
    static int cached[64];
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 256;
    if (cached[d] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0) n = 256;
        cached[d] = n;
    }
    return cached[d];
}

// ------------------------------------------------------- ragged operands
// Shapes off the 16-byte grid (K or N not a multiple of 16) and operands
// not 16-byte aligned cannot be moved by whole 16-byte chunks: rows start at
// unaligned offsets, and a chunk that runs past the end of a buffer cannot be
// range-checked byte by byte.  Such operands are repacked once into
// zero-padded, aligned panels A' [Mp][Kp] and B' [Kp][Np] (M, K, N rounded
// up to 256) in the workspace, and the full-tile kernels run on those with
// C's own row stride and row / column bounds.  The padding is zero on both sides of
// every product, so C is unchanged.  One launch for both operands
// (blockIdx.z), or for B alone when A already suits the full-tile kernels
// (16-byte aligned, M % 128 == 0, K % 256 == 0: B' is [K][Np] and A is used
// in place); each thread writes 16 bytes of each of PAD_ROWS panel rows.  A wave's 64 output
// chunks start at one byte offset sh (0..15) into the 16-byte grid of the
// source, so each lane loads the aligned chunk under its own (lane 63 also the
// one after the wave's span), takes its neighbour's from lane + 1 and
// funnel-shifts the pair by sh.  Chunks that reach past either end of the
// source buffer are read byte by byte, so no load leaves the buffer.
constexpr int PAD_ROWS = 2;   // panel rows per thread and pass
__device__ inline uint4 pad_load16(const int8_t *src, long long o, long long total) {
    if (o >= 0 && o + 16 <= total) return *(const uint4 *)(src + o);
    uint32_t w[4] = {0, 0, 0, 0};
    for (int e = 0; e < 16; ++e)
        if (o + e >= 0 && o + e < total) w[e >> 2] |= (uint32_t)(uint8_t)src[o + e] << (8 * (e & 3));
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ __launch_bounds__(256) void pad_i8_kernel(const int8_t *__restrict__ A, const int8_t *__restrict__ B,
                                                     int M, int N, int K, int Mp, int Kp, int Np,
                                                     uint4 *__restrict__ Ap, uint4 *__restrict__ Bp, int zb) {
    const bool is_b = (int)blockIdx.z == zb;   // zb = 1: A at z = 0, B at z = 1; zb = 0: B only
    const int8_t *src = is_b ? B : A;
    uint4 *dst = is_b ? Bp : Ap;
    const int rows = is_b ? K : M, rows_out = is_b ? Kp : Mp, cols = is_b ? N : K, dcols = is_b ? Np : Kp;
    const long long total = (long long)rows * cols;
    const int lane = threadIdx.x & 63;
    const int c0 = (blockIdx.x * 256 + threadIdx.x) * 16, cw = c0 - 16 * lane;   // cw: the wave's first column
    if (cw >= dcols) return;   // uniform per wave
    // PAD_ROWS rows per pass, their loads issued before any is used
    for (int r0 = blockIdx.y * PAD_ROWS; r0 < rows_out; r0 += gridDim.y * PAD_ROWS) {
        uint4 q[PAD_ROWS], q63[PAD_ROWS];
        int sh[PAD_ROWS];
#pragma unroll
        for (int r = 0; r < PAD_ROWS; ++r) {
            const int row = r0 + r;
            q[r] = q63[r] = make_uint4(0, 0, 0, 0);
            sh[r] = 0;
            if (row < rows && cw < cols) {
                const long long p = (long long)row * cols + cw;
                sh[r] = (int)(((uintptr_t)src + (uintptr_t)p) & 15);
                const long long o = p - sh[r];   // lane 0's aligned chunk, relative to src
                q[r] = pad_load16(src, o + 16 * lane, total);
                if (lane == 63) q63[r] = pad_load16(src, o + 16 * 64, total);
            }
        }
#pragma unroll
        for (int r = 0; r < PAD_ROWS; ++r) {
            const int row = r0 + r;
            uint32_t w[4] = {0, 0, 0, 0};
            if (row < rows && cw < cols) {   // uniform per wave: every lane takes part in the shuffles
                uint4 n;
                n.x = (uint32_t)__shfl_down((int)q[r].x, 1);
                n.y = (uint32_t)__shfl_down((int)q[r].y, 1);
                n.z = (uint32_t)__shfl_down((int)q[r].z, 1);
                n.w = (uint32_t)__shfl_down((int)q[r].w, 1);
                if (lane == 63) n = q63[r];
                const uint32_t x[8] = {q[r].x, q[r].y, q[r].z, q[r].w, n.x, n.y, n.z, n.w};
                const int s4 = sh[r] >> 2, sb = sh[r] & 3;
                uint32_t y[5];
#pragma unroll
                for (int i = 0; i < 5; ++i)
                    y[i] = s4 == 0 ? x[i] : s4 == 1 ? x[i + 1] : s4 == 2 ? x[i + 2] : x[i + 3];
#pragma unroll
                for (int i = 0; i < 4; ++i) w[i] = __builtin_amdgcn_alignbyte(y[i + 1], y[i], sb);
                const int valid = cols - c0;   // bytes of this chunk inside the row
                if (valid < 16) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int v = valid - 4 * i;
                        w[i] = v <= 0 ? 0u : v >= 4 ? w[i] : w[i] & ((1u << (8 * v)) - 1u);
                    }
                }
            }
            if (row < rows_out && c0 < dcols)
                dst[((long long)row * dcols + c0) >> 4] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

static bool i8_fast(const int8_t *A, const int8_t *B, int M, int N, int K) {
    return (K % 16 == 0) && (N % 16 == 0) && (((uintptr_t)A & 15) == 0) && (((uintptr_t)B & 15) == 0) &&
           (size_t)M * K < 0x80000000ull && (size_t)K * N < 0x80000000ull;
}

// Workspace of the repack path: 0 when the operands go to the kernels as
// they are (16-byte grid, or panels beyond the buffer fast paths' 2 GiB).
static inline size_t round256(size_t x) { return (x + 255) / 256 * 256; }
// Shapes on the 16-byte grid that no 128-row kernel takes go to the
// 256 x 256 edge kernel; when its grid would not fill one round of the chip
// (1008^3: 16 tiles, 17.2 us) the padded panels are faster (1024^3 panels on
// 128 x 128 tiles: 6 us + the repack), so they are repacked as well -- but
// only where the padding is small: M and N at least 256 and no dimension
// grown by more than 1/8 (496 -> 512, 1008 -> 1024, 2000 -> 2048), so small
// shapes such as the reference sweep's 16^3 .. 256^3 stay on the edge kernel
// with no workspace, and the panels stay within 27/64 more bytes than the
// operands.
static bool i8_pad_small(int d) { return round256(d) * 8 <= (size_t)d * 9; }
static bool i8_edge_underfills(int M, int N, int K) {
    const int cus = cu_count();
    if (M < 256 || N < 256 || !i8_pad_small(M) || !i8_pad_small(N) || !i8_pad_small(K)) return false;
    const bool full128 = M % 128 == 0 && N % 256 == 0 && K % 128 == 0;
    const bool one128 = M % 128 == 0 && N % 128 == 0 && K % 128 == 0 && (long long)(M / 128) * (N / 128) <= cus;
    // ... and only when the panels fit one round of 128 x 128 tiles (3000 x
    // 3008^2 on its 144 edge tiles: 36.6 us; on 3072-wide panels, two rounds
    // of persistent 128 x 256 tiles: 54.6 us)
    return !full128 && !one128 && (long long)((M + 255) / 256) * ((N + 255) / 256) < cus &&
           (long long)(round256(M) / 128) * (long long)(round256(N) / 128) <= cus;
}

size_t i8_workspace_bytes(int M, int N, int K, bool aligned) {
    if (i8_small(M, N, K)) return 0;
    const size_t Mp = round256(M), Kp = round256(K), Np = round256(N);
    const bool grid16 = K % 16 == 0 && N % 16 == 0 && aligned;
    if (K == 0 || Mp * Kp >= 0x80000000ull || Kp * Np >= 0x80000000ull) return 0;
    if (grid16 && !i8_edge_underfills(M, N, K)) return 0;
    return Mp * Kp + Kp * Np;
}

// Operands on the 16-byte grid: pick the kernel; C has row stride ldc and
// rows < mst, columns < nst are stored (masked only when that is not the
// whole M x N).
static void launch_i8_on_grid(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, int ldc, int mst,
                              int nst, hipStream_t s) {
    const bool mask = mst != M || nst != N || ldc != N;
    using namespace i8g;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const dim3 grid(tiles_m * tiles_n), block(THREADS);
    const bool full128 = K > 0 && M % h128::BM == 0 && N % BN == 0 && K % h128::KS == 0;
    const bool full128n = K > 0 && M % h128::BM == 0 && N % 128 == 0 && K % h128::KS == 0;
    const int cus = cu_count(), tm128 = M / h128::BM;
    // 128 x 128 tiles when they fit one round of the chip (M N <= 2^22 on 256
    // CUs: 128 x 256 tiles would leave half the CUs idle); otherwise 256 x 256
    // tiles when they fill their rounds (below), else the persistent
    // 128 x 256 tiles whenever the shape allows them; the rest go to the
    // range-checked 256 x 256 kernel
    const bool use128n = full128n && tm128 * (N / 128) <= cus;
    // 256 x 256 tiles (faster K loop, stores not overlapped) when they fill
    // their rounds of the chip to at least 7/8 (4096^3 and 8192^3: exactly,
    // the MLP layer: 688 tiles, 0.9 of three rounds; not 6144^3: 576 tiles,
    // 0.75 of three rounds, where the persistent 128 x 256 tiles balance
    // better)
    const int t256n = (M / t256::BM) * (N / t256::TN), r256 = (t256n + cus - 1) / cus;
    const bool use256 = !use128n && K > 0 && M % t256::BM == 0 && N % t256::TN == 0 && K % (BK * t256::NST) == 0 &&
                        t256n >= cus && 8 * t256n >= 7 * r256 * cus;
    const bool use128 = !use128n && !use256 && full128;
    if (use256) {
        const int tm = M / t256::BM, tn = N / t256::TN, gm = t256::group_m(r256);
        if (mask)
            hipLaunchKernelGGL(t256::gemm_i8_t256_kernel<true>, dim3(tm * tn), block, 0, s, A, B, C, M, N, K, tm, tn,
                               ldc, mst, nst, gm, I16Epi{});
        else
            hipLaunchKernelGGL(t256::gemm_i8_t256_kernel<false>, dim3(tm * tn), block, 0, s, A, B, C, M, N, K, tm, tn,
                               ldc, mst, nst, gm, I16Epi{});
    } else if (use128 || use128n) {
        const int tn = use128n ? N / 128 : N / BN, nt = tm128 * tn;
        // persistent workgroups: as many rounds of tiles as the CUs need, the
        // tiles spread evenly over a multiple of 8 workgroups (one XCD each)
        const int rounds = (nt + cus - 1) / cus;
        const int wgs = rounds == 1 ? nt : ((nt + rounds - 1) / rounds + 7) / 8 * 8;
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(wgs), block, 0, s, A, B, C, M, N, K, tm128, tn, ldc, mst, nst,
                               h128::group_m(use128n));
        };
        using namespace h128;
        if (use128n) {   // one round by construction
            if (mask) go(gemm_i8_h128_kernel<true, false, 128>);
            else go(gemm_i8_h128_kernel<false, false, 128>);
        } else {
            if (mask) rounds > 1 ? go(gemm_i8_h128_kernel<true, true, 256>) : go(gemm_i8_h128_kernel<true, false, 256>);
            else rounds > 1 ? go(gemm_i8_h128_kernel<false, true, 256>) : go(gemm_i8_h128_kernel<false, false, 256>);
        }
    } else {
        hipLaunchKernelGGL((gemm_i8_dma_kernel<EPI_I8, false>), grid, block, 0, s, A, B, C, M, N, K, tiles_m, tiles_n,
                           ldc, mst, nst, I16Epi{});
    }
}

hipError_t launch_gemm_i8(const int8_t *A, const int8_t *B, int32_t *C, int M, int N, int K, void *ws,
                          hipStream_t s) {
    using namespace i8g;
    if (i8_small(M, N, K)) return launch_gemm_i8_small(A, B, C, M, N, K, s);
    const bool aligned = (((uintptr_t)A & 15) == 0) && (((uintptr_t)B & 15) == 0);
    const size_t pad = i8_workspace_bytes(M, N, K, aligned);
    if (i8_fast(A, B, M, N, K) && !(pad && ws)) {
        launch_i8_on_grid(A, B, C, M, N, K, N, M, N, s);
    } else if (pad && ws) {
        const int Mp = (int)round256(M), Kp = (int)round256(K), Np = (int)round256(N);
        if (((uintptr_t)A & 15) == 0 && M % 128 == 0 && K % 256 == 0) {
            // A already suits the full-tile kernels (a ragged or misaligned B,
            // e.g. N = 1000): repack only B into [K][Np] panels
            int8_t *Bp = (int8_t *)ws;
            const int ry = (K + PAD_ROWS - 1) / PAD_ROWS;
            const dim3 pgrid((unsigned)((Np / 16 + 255) / 256), (unsigned)(ry < 65535 ? ry : 65535), 1);
            hipLaunchKernelGGL(pad_i8_kernel, pgrid, dim3(256), 0, s, A, B, M, N, K, M, K, Np, (uint4 *)nullptr,
                               (uint4 *)Bp, 0);
            launch_i8_on_grid(A, Bp, C, M, Np, K, N, M, N, s);
            return hipGetLastError();
        }
        int8_t *Ap = (int8_t *)ws;
        int8_t *Bp = Ap + (size_t)Mp * Kp;
        const int wide = Kp > Np ? Kp : Np, tall = Mp > Kp ? Mp : Kp;
        const int ry = (tall + PAD_ROWS - 1) / PAD_ROWS;
        const dim3 pgrid((unsigned)((wide / 16 + 255) / 256), (unsigned)(ry < 65535 ? ry : 65535), 2);
        hipLaunchKernelGGL(pad_i8_kernel, pgrid, dim3(256), 0, s, A, B, M, N, K, Mp, Kp, Np, (uint4 *)Ap,
                           (uint4 *)Bp, 1);
        launch_i8_on_grid(Ap, Bp, C, Mp, Np, Kp, N, M, N, s);
    } else {
        const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
        hipLaunchKernelGGL(gemm_i8_kernel<false>, dim3(tiles_m * tiles_n), dim3(THREADS), 0, s, A, B, C, M, N, K,
                           tiles_m, tiles_n);
    }
    return hipGetLastError();
}

// int16 GEMM through the int8 DMA kernel on the limb interleave (see
// det_gemm_i16x.hip): A2 [2*M16][Kp], B2 [Kp][N2] with Kp % 16 == 0,
// N2 % 16 == 0, both 16-byte aligned, 2*M16*Kp and Kp*N2 below 2^31.
hipError_t launch_gemm_i8_i16epi(const int8_t *A2, const int8_t *B2, int M2, int N2, int Kp, const uint32_t *rowsum,
                                 const uint32_t *colsum, int ncs, int32_t *C, int M16, int N16, int K16,
                                 hipStream_t s) {
    using namespace i8g;
    const int tiles_m = (M2 + BM - 1) / BM, tiles_n = (N2 + BN - 1) / BN;
    I16Epi e{rowsum, colsum, C, M16, N16, ncs, 0x80u, (uint32_t)((uint64_t)(uint32_t)K16 * 0x4000u)};
    const bool full = Kp > 0 && M2 % BM == 0 && N2 % BN == 0 && Kp % (BK * NSTAGE) == 0;
    // 16x16x64 256 x 256 tiles when they fill whole rounds, as for int8
    const int cus = cu_count(), nt = tiles_m * tiles_n, rounds = (nt + cus - 1) / cus;
    if (full && nt >= cus && 8 * nt >= 7 * rounds * cus)
        hipLaunchKernelGGL((t256::gemm_i8_t256_kernel<false, EPI_I16>), dim3(nt), dim3(THREADS), 0, s, A2, B2,
                           (int32_t *)nullptr, M2, N2, Kp, tiles_m, tiles_n, N2, M2, N2, t256::group_m(rounds), e);
    else if (full)
        hipLaunchKernelGGL((gemm_i8_dma_kernel<EPI_I16, true>), dim3(tiles_m * tiles_n), dim3(THREADS), 0, s, A2, B2,
                           (int32_t *)nullptr, M2, N2, Kp, tiles_m, tiles_n, N2, M2, N2, e);
    else
        hipLaunchKernelGGL((gemm_i8_dma_kernel<EPI_I16, false>), dim3(tiles_m * tiles_n), dim3(THREADS), 0, s, A2, B2,
                           (int32_t *)nullptr, M2, N2, Kp, tiles_m, tiles_n, N2, M2, N2, e);
    return hipGetLastError();
}

}  // namespace det
