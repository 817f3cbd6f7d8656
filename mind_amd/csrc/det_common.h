// det_common.h -- shared definitions for the gfx950 deterministic integer
// GEMM / GEMV kernels and their C-ABI host layer.
//
// Every kernel in this library is integer-only: int8 MFMA with i32
// accumulation, 32/64-bit VALU integer arithmetic, no floating point anywhere.
// Integer addition is associative, so every reduction order gives the same
// bits; determinism does not depend on launch shape or scheduling.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace det {

typedef long v2i64 __attribute__((ext_vector_type(2)));
typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef short v2i16 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- MFMA
// v_mfma_i32_16x16x64_i8: D[16x16] += A[16x64] * B[64x16], int8 in, i32 out.
// Operand layout (per lane l, 16 bytes): A row (l & 15), B column (l & 15),
// K slice selected by l >> 4 (the hardware assigns the same K index to the
// same (lane group, byte) position of A and B, so any consistent per-lane K
// slicing of the two operands yields the exact dot product).
// Result layout: lane l, element r holds D[4*(l >> 4) + r][l & 15].
__device__ __forceinline__ v4i32 mfma16x16x64(const v2i64 a, const v2i64 b, v4i32 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// v_mfma_i32_32x32x32_i8: D[32x32] += A[32x32] * B[32x32].  Operands: lane l
// holds 16 bytes of A row (l & 31) / B column (l & 31), K slice l >> 5.
// Result: lane l, element r holds D[8*(r >> 2) + 4*(l >> 5) + (r & 3)][l & 31].
typedef int v16i32 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ v16i32 mfma32x32x32(const v2i64 a, const v2i64 b, v16i32 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- bytes
// perm(hi, lo, sel): byte i of the result is byte sel.byte[i] of the 64-bit
// value {hi:lo} (0..3 = lo bytes, 4..7 = hi bytes).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4x4 byte transpose: input d[r] holds row r (bytes = columns 0..3), output
// e[c] holds column c (bytes = rows 0..3).
__device__ __forceinline__ void transpose4x4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                                             uint32_t &e0, uint32_t &e1, uint32_t &e2, uint32_t &e3) {
    const uint32_t t0 = perm(d1, d0, 0x06020400u);  // d0.b0 d1.b0 d0.b2 d1.b2
    const uint32_t t1 = perm(d1, d0, 0x07030501u);  // d0.b1 d1.b1 d0.b3 d1.b3
    const uint32_t t2 = perm(d3, d2, 0x06020400u);  // d2.b0 d3.b0 d2.b2 d3.b2
    const uint32_t t3 = perm(d3, d2, 0x07030501u);  // d2.b1 d3.b1 d2.b3 d3.b3
    e0 = perm(t2, t0, 0x05040100u);                 // col 0
    e1 = perm(t3, t1, 0x05040100u);                 // col 1
    e2 = perm(t2, t0, 0x07060302u);                 // col 2
    e3 = perm(t3, t1, 0x07060302u);                 // col 3
}

// 8x8 byte transpose of a block held as 8 rows x 2 dwords (lo = columns
// 0..3, hi = columns 4..7).  Output: 8 columns x 2 dwords (lo = rows 0..3,
// hi = rows 4..7).
__device__ __forceinline__ void transpose8x8(const uint32_t (&lo)[8], const uint32_t (&hi)[8],
                                             uint32_t (&clo)[8], uint32_t (&chi)[8]) {
    transpose4x4(lo[0], lo[1], lo[2], lo[3], clo[0], clo[1], clo[2], clo[3]);
    transpose4x4(hi[0], hi[1], hi[2], hi[3], clo[4], clo[5], clo[6], clo[7]);
    transpose4x4(lo[4], lo[5], lo[6], lo[7], chi[0], chi[1], chi[2], chi[3]);
    transpose4x4(hi[4], hi[5], hi[6], hi[7], chi[4], chi[5], chi[6], chi[7]);
}

// ---------------------------------------------------------------- buffers
// Raw buffer resource over [base, base + bytes): a buffer load whose offset
// lies outside returns zero without touching memory, so tile edges need no
// branches (an invalid lane passes OOB_OFFSET).  Requires bytes < 2^31.
constexpr uint32_t OOB_OFFSET = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const v4i32 v = __builtin_bit_cast(v4i32, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
// The same with a uniform byte offset in soffset (not range-checked: voff +
// soff must lie inside the buffer).
__device__ __forceinline__ uint4 buf_load16s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const v4i32 v = __builtin_bit_cast(v4i32, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// ---------------------------------------------------------------- XCD map
// Workgroups are dealt round-robin to the 8 XCDs (each with its own L2).
// Remap the hardware workgroup id so that each XCD receives a contiguous run
// of logical tile ids: neighbouring tiles, which share A rows / B columns,
// then hit the same L2.
__device__ __forceinline__ int xcd_remap(int wg, int nwg) {
    constexpr int XCD = 8;
    const int per = nwg / XCD;           // full rounds
    const int rem = nwg - per * XCD;     // leftover workgroups in the last round
    const int x = wg % XCD, slot = wg / XCD;
    if (slot < per) return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + slot;
    return x * (per + 1) + per;          // x < rem here
}

// ---------------------------------------------------------------- LDS DMA
typedef __attribute__((address_space(3))) int8_t *lds_i8_ptr;

// Raw buffer descriptor as four SGPR words (base, stride 0, num_records,
// gfx9 data-format word) for the inline-assembly DMA below.  bytes < 2^31.
__device__ __forceinline__ v4i32 rsrc_words(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return (v4i32){(int)(uint32_t)a, (int)(uint32_t)(a >> 32) & 0xffff, (int)bytes, 0x00020000};
}
// One buffer_load_dwordx4 ... lds: lane i's 16 bytes at `voff` land at LDS
// byte lds + 16 i (an offset past num_records lands zeros).  The LDS DMA
// reads M0 one wait state after the SALU write at the earliest (the
// compiler keeps the same distance for its own LDS DMA), hence the s_nop;
// the compiler's hazard pass does not look inside inline assembly.  Written as
// inline assembly so the compiler's wait-count pass does not treat every
// later LDS read as dependent on it (it would drain all loads in flight); a
// kernel using it orders these loads itself with explicit s_waitcnt vmcnt
// and s_barrier, and issues no other vector-memory loads while they are
// outstanding.
__device__ __forceinline__ void dma16(v4i32 rsrc, uint32_t lds, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}
// The same with a uniform byte offset added from an SGPR (soffset), so a
// loop can advance every lane's address without a vector add.  The range
// check covers voffset only: soffset is added after it, so voff + soff must
// itself stay inside the buffer (an out-of-range soffset is a real access,
// not a zero fill).
__device__ __forceinline__ void dma16s(v4i32 rsrc, uint32_t lds, int voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_i8_ptr)(const int8_t *)(p));
}

}  // namespace det

// s_waitcnt with vmcnt <= n (n < 64), expcnt / lgkmcnt left unconstrained.
#define DET_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
// s_waitcnt lgkmcnt(0) only.
#define DET_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xc07f & ~(15 << 8))

// Host-side launch check shared by the entry points.
#define DET_HIP_CHECK(expr)                                      \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return det_fail_hip(_e, #expr);    \
    } while (0)

extern "C" int64_t det_fail_hip(hipError_t e, const char *what);
extern "C" int64_t det_fail(int64_t code, const char *msg);
