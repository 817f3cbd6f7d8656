// det_gemv_mfma.hip -- exact Q16.16 GEMV for several query vectors at once:
// S on the int8 MFMA, the per-term residue on the VALU.
//
//   y[b][i] = (int32) sum_k ( (int64)W[i,k] * (int64)x[b][k]  >>arith 16 ),  b < nb <= 8
// (the batched form of __mind_blas_gemv_q16_mt: reference src/mlir/lowering.rs:
// 9822-9997; oracle benches/det_gemv_q16_mt.rs:186-197).
//
// Why: the one-vector kernel (det_gemv.hip) spends ~8 VALU slots per term on
// the 64-bit product; with 8 vectors that is ~4x the VALU budget HBM speed
// allows.  Here, per W element, the VALU only splits W into limbs and
// computes the residue for each vector (1 op per term):
//   * S = sum_k W x exactly (mod 2^48) from int8 limb-pair MFMAs.  W is
//     written as signed int8 limbs t_p (low bytes biased by -128 = u ^ 0x80,
//     c = 0x808080): W = sum_p 2^(8p) t_p + c.  The query vectors (small,
//     prepared once) are written in five balanced base-256 digits
//     d_q in [-128, 127]: x = sum_q 2^(8q) d_q.  Then
//         sum_k W x = sum_{p,q} 2^(8(p+q)) sum_k t_p d_q + c sum_k x,
//     and only pairs with p + q <= 5 matter mod 2^48.  The sum of x is exact
//     and cheap (prep); no row sums of W are needed.
//     v_mfma_i32_16x16x64_i8 takes 16 W rows as A and two digits of the 8
//     query vectors as the 16 B columns (columns 0-7: digit 2Q, 8-15: digit
//     2Q + 1), so 10 MFMAs per 64-wide K step cover every needed pair.
//   * R = sum_k ((W x) mod 2^16) = sum_k ((lo16 W * lo16 x) mod 2^16) with
//     v_pk_mul_lo_u16 + v_dot2_u32_u16 (two terms per pair of ops).
//   * y = (int32)(((S - R) mod 2^48) >> 16).
// Exactness bounds: K <= 32768 keeps the shift-0 and shift-1 partial sums
// (|t_p d_q| <= 2^14) below 2^31 and R below 2^32; shifts >= 2 only need
// their value mod 2^32 (i32 wrap-around).
//
// Layout: a prep kernel rewrites the (small) query vectors into MFMA B
// operands (xp) and packed low halves (xl) in exactly the per-lane K order
// the main kernel uses, chunk by chunk as the main kernel stages them; W is
// streamed once, straight from HBM into registers (buffer loads four K
// steps ahead), and split into limb planes with v_perm.
// Lane l of a wave handles W row (l & 15) and, within each 64-wide K step,
// the K indices {16 j + 4 (l >> 4) + e : j, e < 4}; any consistent K order
// of the A and B operands gives the exact dot product.
#include "det_common.h"
#include "det_kernels.h"

namespace det {
namespace gemv8 {

constexpr int DEPTH = 4;
constexpr uint32_t BIAS4 = 0x80808080u;
constexpr int NQ = 3;                                   // B operands per K step: digit pairs (0,1), (2,3), (4,-)
constexpr int CH = 4;                                   // K steps per LDS chunk (per half)
constexpr int XP_CH = CH * NQ * 64, XL_CH = CH * 64;    // uint4 per chunk
constexpr int X_CH = XP_CH + XL_CH;                     // 1024 uint4 = 16 KiB per chunk

// One 128-thread block per 64-wide K step s, all in registers: thread t
// takes vector v = t >> 4 and the four K indices 16 j + 4 g + e (j = (t >> 2)
// & 3, g = t & 3, e < 4) of the step.  The balanced digits need no loop:
// with u = x + 0x8080808080 (exact in int64), digit q of x is byte q of u
// minus 128, i.e. byte q of u XOR 0x80 read as int8 (adding 128 to every
// digit position turns the balanced digits into the plain base-256 digits
// of u).  A 4 x 4 byte transpose of the four u's low words gives digit words
// 0-3 of this thread's slot, their high words' low bytes digit 4.  The
// step's column sums part[s][v] (exact, int64; summed by the main kernel:
// no atomics, nothing to zero) come from a shuffle reduction over the 16
// threads of each vector.  Vectors v >= nb read as zero (all digits zero).
// Output layout, chunk by chunk (chunk c = steps CH c .. CH c + CH - 1, X_CH
// uint4): xp entries (d8, Q, lane) at (d8 NQ + Q) 64 + lane, lane = b + 16 g,
// column b = v + 8 (q & 1) for digit q = 2 Q + (b >> 3), word j; then xl
// entries at XP_CH + d8 64 + ((j 4 + bp) 4 + g), vector 2 bp + h in its
// dwords 2 h, 2 h + 1.
__global__ __launch_bounds__(128) void prep_kernel(const int32_t *__restrict__ X, int nb, int K,
                                                   uint4 *__restrict__ xw, long long *__restrict__ part) {
    const int s = blockIdx.x, t = threadIdx.x;
    const int v = t >> 4, j = (t >> 2) & 3, g = t & 3;
    const int d8 = s % CH;
    uint32_t *xc = (uint32_t *)(xw + (size_t)(s / CH) * X_CH);
    int32_t x[4] = {0, 0, 0, 0};
    if (v < nb) {
        const int32_t *src = X + (size_t)v * K + 64 * s + 16 * j + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = src[e];
    }
    uint32_t lo[4], hi4 = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const unsigned long long u = (unsigned long long)(long long)x[e] + 0x8080808080ull;
        lo[e] = (uint32_t)u;
        hi4 |= ((uint32_t)(u >> 32) & 0xffu) << (8 * e);
    }
    uint32_t w[5];
    transpose4x4(lo[0], lo[1], lo[2], lo[3], w[0], w[1], w[2], w[3]);
    w[4] = hi4;
#pragma unroll
    for (int q = 0; q < 5; ++q) {
        const int Q = q >> 1, b = v + 8 * (q & 1);
        xc[((d8 * NQ + Q) * 64 + b + 16 * g) * 4 + j] = w[q] ^ BIAS4;
    }
    xc[((d8 * NQ + 2) * 64 + v + 8 + 16 * g) * 4 + j] = 0u;   // digit 5: none
    // low halves: vector v's two K pairs into half h = v & 1 of entry (j, bp = v >> 1, g)
    const uint32_t l01 = ((uint32_t)x[0] & 0xffffu) | ((uint32_t)x[1] << 16);
    const uint32_t l23 = ((uint32_t)x[2] & 0xffffu) | ((uint32_t)x[3] << 16);
    *(uint2 *)(xc + (XP_CH + d8 * 64 + ((j * 4 + (v >> 1)) * 4 + g)) * 4 + 2 * (v & 1)) = make_uint2(l01, l23);
    // exact column sum of vector v over this step: the 16 threads t with t >> 4 == v
    long long cs = (long long)x[0] + x[1] + x[2] + x[3];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) cs += __shfl_xor(cs, o);
    if ((t & 15) == 0) part[(size_t)s * 8 + v] = cs;
}

// One block = 8 waves (2 per SIMD, so one wave's LDS / MFMA latency hides
// behind the other's VALU work) on 64 W rows: wave w takes rows
// 16 (w & 3) .. +16 and K half (w >> 2).  The query operands of a chunk of CH
// K steps of both halves (xp: 3 KiB per step, xl: 1 KiB per step) are staged
// in LDS, double buffered, by all threads through registers: LDS reads wait
// on lgkmcnt, so the only vector-memory loads a step waits for are its own W
// rows, kept DEPTH steps ahead in a register ring (vmcnt retires in order,
// so mixing other loads into that stream would drain the ring).  The staging
// loads of chunk c+1 are issued at the start of chunk c and written to LDS
// at its end.  The two K halves are combined exactly at the end (int64 for
// the shift-0/1 sums).
// Requires K % 512 == 0, K <= 32768, W < 2^31 bytes, nb <= 8.
constexpr int WAVES = 8, THREADS8 = WAVES * 64;
constexpr int STAGE_PER_THREAD = 2 * X_CH / THREADS8;  // 4
struct Tail {                                           // post-loop reduction (aliases the staging)
    int32_t acc[WAVES][6][16][17];
    uint32_t r[WAVES][16][8];
};
constexpr int SMEM_BYTES = sizeof(Tail) > 2 * 2 * X_CH * 16 ? sizeof(Tail) : 2 * 2 * X_CH * 16;

__global__ __launch_bounds__(THREADS8, 1) void gemv8_kernel(const int32_t *__restrict__ W,
                                                            const uint4 *__restrict__ xw,
                                                            const long long *__restrict__ part,
                                                            int32_t *__restrict__ Y, int M, int K, int nb) {
    __shared__ __attribute__((aligned(16))) char smem[SMEM_BYTES];
    uint4 *s_x = (uint4 *)smem;                       // [2 buffers][2 halves][X_CH]
    Tail &tail = *(Tail *)smem;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int rg = wave & 3, kh = __builtin_amdgcn_readfirstlane(wave >> 2);
    const int row0 = blockIdx.x * 64 + rg * 16;
    const int myrow = min(row0 + r, M - 1);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(W, (uint32_t)M * (uint32_t)K * 4u);
    const int nsteps = K / 64, half = nsteps / 2, nch = half / CH;
    const int sbeg = kh * half;
    const uint32_t wbase = ((uint32_t)myrow * (uint32_t)K + 4u * g) * 4u;   // bytes

    // staging of chunk c of both halves: 2 X_CH uint4, slot i of thread tid
    // = entry f = i THREADS8 + tid, half f / X_CH (global chunk c, or
    // half / CH + c), entry f % X_CH of that chunk.  One buffer resource over
    // all chunks; buffer loads with 32-bit offsets keep the address registers
    // apart from the data, so the loads stay in flight (the wait is at the
    // LDS store at the end of the chunk).
    static_assert(STAGE_PER_THREAD == 4 && X_CH == 2 * THREADS8, "staging slots");
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xw, (uint32_t)(K / 64 / CH) * X_CH * 16u);
    uint4 stg[STAGE_PER_THREAD];
    auto stage_load = [&](int c) {
        const uint32_t c0 = (uint32_t)c, c1 = (uint32_t)(half / CH + c);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            stg[i] = buf_load16(rx, ((c0 * X_CH) + i * THREADS8 + tid) * 16u);
            stg[2 + i] = buf_load16(rx, ((c1 * X_CH) + i * THREADS8 + tid) * 16u);
        }
    };
    auto stage_store = [&](int buf) {
        uint4 *d = s_x + buf * 2 * X_CH;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            d[i * THREADS8 + tid] = stg[i];
            d[X_CH + i * THREADS8 + tid] = stg[2 + i];
        }
    };

    v4i32 acc[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) acc[i] = (v4i32){0, 0, 0, 0};
    uint32_t racc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) racc[b] = 0;

    // prologue: W ring, chunk-0 staging and the column-sum partials all in
    // flight together (one memory round trip)
    uint4 wb[DEPTH][4];   // W ring: DEPTH steps in flight; loads past the end read out of range
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
#pragma unroll
        for (int j = 0; j < 4; ++j) wb[d][j] = buf_load16s(rw, wbase + 64u * j, (uint32_t)(256 * (sbeg + d)));
    stage_load(0);
    // column sums of the query vectors: thread t adds the per-step partials
    // i = t/8 + 64 u (u < 8, K <= 32768) of vector t % 8 (finished in the tail)
    long long pv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = (tid >> 3) + 64 * u;
        pv[u] = i < 2 * half ? part[(size_t)i * 8 + (tid & 7)] : 0;
    }
    long long cpart = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) cpart += pv[u];
    stage_store(0);
    __syncthreads();

    for (int c = 0; c < nch; ++c) {
        const int buf = c & 1;
        stage_load(c + 1 < nch ? c + 1 : c);   // branch-free; the last reload is unused
        __builtin_amdgcn_sched_barrier(0);      // keep its LDS stores at the end of the chunk
        const uint4 *sxp = s_x + (buf * 2 + kh) * X_CH;
        const uint4 *sxl = sxp + XP_CH;
#pragma unroll
        for (int d8 = 0; d8 < CH; ++d8) {
            const int d = d8 % DEPTH;
            const int ls = c * CH + d8;         // step within this wave's half
            const int st = sbeg + ls;
            // consume the ring slot (limb transpose, low halves) before
            // reloading it: the reload then reuses the same registers, so no
            // register copy has to wait for a load still in flight.  The
            // bias goes on after the transpose: planes 0-2 only.  The reload
            // is DEPTH steps ahead; past the half's end it re-reads the half's
            // last step (never consumed), so every load stays inside this
            // lane's W row: the step offset goes through the uniform soffset,
            // which the range check does not cover
            const uint32_t wsoff = (uint32_t)(256 * min(st + DEPTH, sbeg + half - 1));
            uint32_t T[4][4], L[4][2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint4 w = wb[d][j];
                transpose4x4(w.x, w.y, w.z, w.w, T[j][0], T[j][1], T[j][2], T[j][3]);
#pragma unroll
                for (int pl = 0; pl < 3; ++pl) T[j][pl] ^= BIAS4;
                L[j][0] = perm(w.y, w.x, 0x05040100u);   // lo16 of K e=0,1
                L[j][1] = perm(w.w, w.z, 0x05040100u);   // lo16 of K e=2,3
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                wb[d][j] = buf_load16s(rw, wbase + 64u * j, wsoff);
            // query low halves of this step: the first half is read here, so
            // its LDS latency hides behind the MFMAs, the second half after
            // them, behind the first half's residues (reading each at its
            // point of use made the compiler wait on every read: 16 LDS round
            // trips per step in series)
            uint4 XV[4][4];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int bp = 0; bp < 4; ++bp) XV[j][bp] = sxl[((d8 * 4 + j) * 4 + bp) * 4 + g];
            v2i64 B[NQ];
#pragma unroll
            for (int q = 0; q < NQ; ++q) B[q] = __builtin_bit_cast(v2i64, sxp[(d8 * NQ + q) * 64 + lane]);
            // A operands: W limb planes t_p for 16 K; B operand Q holds digits
            // 2Q (columns 0-7) and 2Q + 1 (8-15): accumulator set p + 2Q gets
            // shift p + 2Q in columns 0-7 and p + 2Q + 1 in 8-15
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const v2i64 A = __builtin_bit_cast(v2i64, (v4i32){(int)T[0][p], (int)T[1][p], (int)T[2][p], (int)T[3][p]});
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    if (p + 2 * q <= 5) acc[p + 2 * q] = mfma16x16x64(A, B[q], acc[p + 2 * q]);
            }
            // residues for every query vector
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 2; j < 4; ++j)
#pragma unroll
                for (int bp = 0; bp < 4; ++bp) XV[j][bp] = sxl[((d8 * 4 + j) * 4 + bp) * 4 + g];
            // two 16-bit residues (lo16 w * lo16 x mod 2^16) per
            // v_pk_mul_lo_u16, added into the vector's sum by v_dot2_u32_u16
            // against (1, 1): a K group's 16 products are formed before its
            // 16 sums, so no sum waits on the product just before it
            const v2u16 one = {1, 1};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v2u16 L0 = __builtin_bit_cast(v2u16, L[j][0]), L1 = __builtin_bit_cast(v2u16, L[j][1]);
                v2u16 P[4][4];
#pragma unroll
                for (int bp = 0; bp < 4; ++bp) {
                    const uint4 xv = XV[j][bp];
                    P[bp][0] = L0 * __builtin_bit_cast(v2u16, xv.x);
                    P[bp][1] = L1 * __builtin_bit_cast(v2u16, xv.y);
                    P[bp][2] = L0 * __builtin_bit_cast(v2u16, xv.z);
                    P[bp][3] = L1 * __builtin_bit_cast(v2u16, xv.w);
                }
#pragma unroll
                for (int bp = 0; bp < 4; ++bp)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t r = __builtin_amdgcn_udot2(P[bp][2 * h], one, racc[2 * bp + h], false);
                        racc[2 * bp + h] = __builtin_amdgcn_udot2(P[bp][2 * h + 1], one, r, false);
                    }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        stage_store(buf ^ 1);   // buffer buf ^ 1 was last read in chunk c - 1
        __syncthreads();
    }

    // residue: sum the four K groups of each row (lanes r, r+16, r+32, r+48)
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        racc[b] += __shfl_xor(racc[b], 16);
        racc[b] += __shfl_xor(racc[b], 32);
    }
    // (the loop ended with a barrier: the staging area is free for the tail)
#pragma unroll
    for (int sft = 0; sft < 6; ++sft)
#pragma unroll
        for (int e = 0; e < 4; ++e) tail.acc[wave][sft][4 * g + e][r] = acc[sft][e];
    if (g == 0)
#pragma unroll
        for (int b = 0; b < 8; ++b) tail.r[wave][r][b] = racc[b];
    // finish the column sums: lanes with equal (lane & 7) within the wave,
    // then the eight waves
    cpart += __shfl_xor(cpart, 8);
    cpart += __shfl_xor(cpart, 16);
    cpart += __shfl_xor(cpart, 32);
    __shared__ long long s_cs[WAVES][8];
    if (lane < 8) s_cs[wave][lane] = cpart;
    __syncthreads();
    // 64 rows x 8 vectors = 512 outputs, one per thread, summing both K halves
    const int rgo = tid >> 7, row = (tid >> 3) & 15, b = tid & 7;
    const int grow = blockIdx.x * 64 + rgo * 16 + row;
    if (b >= nb || grow >= M) return;
    // shift 0: set 0 columns 0-7; shift s >= 1: set s - 1 columns 8-15 plus
    // set s columns 0-7 (exact in int64 for s <= 1, mod 2^32 above)
    long long s0 = 0, s1 = 0;
    uint32_t hi[4] = {0, 0, 0, 0}, rsum = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int wv = h * 4 + rgo;
        s0 += tail.acc[wv][0][row][b];
        s1 += (long long)tail.acc[wv][0][row][8 + b] + tail.acc[wv][1][row][b];
#pragma unroll
        for (int sft = 2; sft < 6; ++sft)
            hi[sft - 2] += (uint32_t)tail.acc[wv][sft - 1][row][8 + b] + (uint32_t)tail.acc[wv][sft][row][b];
        rsum += tail.r[wv][row][b];
    }
    long long colsum_b = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) colsum_b += s_cs[w][b];
    unsigned long long S = 0x808080ull * (unsigned long long)colsum_b;   // c sum_k x
    S += (unsigned long long)s0 + ((unsigned long long)s1 << 8);
#pragma unroll
    for (int sft = 2; sft < 6; ++sft) S += (unsigned long long)hi[sft - 2] << (8 * sft);
    S -= (unsigned long long)rsum;
    Y[(size_t)b * M + grow] = (int32_t)(uint32_t)(S >> 16);
}

}  // namespace gemv8

size_t gemv8_workspace_bytes(int K) {
    return (size_t)K / 64 / gemv8::CH * gemv8::X_CH * 16 + (size_t)K / 64 * 8 * 8;
}

bool gemv8_eligible(const int32_t *W, const int32_t *X, int M, int K) {
    return M >= 16 && K % 512 == 0 && K <= 32768 && (size_t)M * K * 4 < 0x80000000ull &&
           ((uintptr_t)W & 15) == 0 && ((uintptr_t)X & 3) == 0;
}

// X: [nb][K] with nb <= 8, Y: [nb][M].  Requires gemv8_eligible.
hipError_t launch_gemv_q16_mfma(const int32_t *W, const int32_t *X, int32_t *Y, int M, int K, int nb, void *ws,
                                hipStream_t s) {
    using namespace gemv8;
    uint4 *xw = (uint4 *)ws;
    long long *part = (long long *)(xw + (size_t)K / 64 / CH * X_CH);
    hipLaunchKernelGGL(prep_kernel, dim3(K / 64), dim3(128), 0, s, X, nb, K, xw, part);
    hipLaunchKernelGGL(gemv8_kernel, dim3((M + 63) / 64), dim3(THREADS8), 0, s, W, xw, part, Y, M, K, nb);
    return hipGetLastError();
}

}  // namespace det
