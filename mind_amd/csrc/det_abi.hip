// det_abi.hip -- the extern "C" boundary of libmind_det_hip.so.
//
// Three layers, all C-ABI, no torch or HIP types in any signature:
//  1. The reference's own intrinsic symbols with its i64 "Option C" ABI
//     (every pointer passed as int64_t, return 0 on success):
//     __mind_blas_matmul_mm_i8_v, ..._q16_v, gemv, rmajor, dot
//     (arity table: reference src/type_checker/mod.rs:2266-2332).  They take
//     HOST pointers, like the reference, and are synchronous: H2D, kernel,
//     D2H on a library-owned stream, then return.
//  2. The harness symbols the reference benches / gate dlsym (gemmi8,
//     gemmqmm, gemmq, mmq, mmi16, gemvq, dotq...: tests/cross_substrate_
//     identity.rs:70-150, benches/det_*.rs), same ABI.
//  3. det_*: typed C entry points, host-pointer and device-pointer (_dev,
//     asynchronous on a caller stream) forms, plus the small runtime the
//     harness needs (device memory, copies, streams, events, errors).
//
// Errors: the reference's kernels never fail and return 0; here a HIP
// failure or an invalid argument returns a negative code and records a
// message readable through det_last_error() (thread-local), like the
// reference's mind_last_error (src/ffi/mod.rs:173).  A NULL pointer or a
// non-positive size with nothing to compute follows the reference's Track A
// convention and returns 0 (runtime-support/mind_intrinsics.c:1537-1539).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "det_common.h"
#include "det_copy_pool.h"
#include "det_kernels.h"
#include "../../include/mind_det.h"

namespace {

// Last error text of this thread.  A plain buffer, not a std::string: a
// thread_local object with a destructor keeps the library loaded after
// dlclose (the C runtime holds a DSO while it has pending thread-local
// destructors), so its code object and device globals would stay resident.
thread_local char g_err[512];

void put_err(const char *a, const char *b = nullptr) {
    snprintf(g_err, sizeof g_err, "%s%s%s", a, b ? ": " : "", b ? b : "");
}

constexpr int MAX_DEV = 64;
constexpr int64_t DIM_MAX = 0x7fffffff;
// Pinned ring of large host-pointer transfers (see ring_h2d): RING_SLOTS
// chunks of up to RING_CHUNK bytes each.
constexpr int RING_SLOTS = 4;
constexpr size_t RING_CHUNK = 16u << 20;

// Per-device state.  `mu` serialises the host-pointer entry points on that
// device (like the reference's dispatch lock, runtime-support/
// mind_intrinsics.c:1976) and guards growth of the two device arenas.
struct DevState {
    std::mutex mu;
    hipStream_t stream = nullptr;      // library stream for host-pointer calls
    void *io = nullptr;                // staging for host-pointer operands
    size_t io_bytes = 0;
    void *pin = nullptr;               // pinned host staging for small host-pointer calls
    void *pin_dev = nullptr;           // the same memory as the kernels address it
    bool pin_failed = false;           // pinned allocation refused: small calls copy directly
    char *ring = nullptr;              // pinned chunks of large host-pointer transfers
    char *ring_dev = nullptr;          // the same memory as the copy kernels address it
    hipEvent_t ring_ev[RING_SLOTS] = {};   // the last copy that used each chunk
    bool ring_used[RING_SLOTS] = {};
    unsigned ring_next = 0;            // the chunk the next transfer piece takes
    bool ring_failed = false;          // ring allocation refused: large calls copy directly
    void *ws = nullptr;                // limb-GEMM workspace
    size_t ws_bytes = 0;
    hipEvent_t ws_free = nullptr;      // recorded after the last workspace user
};
DevState g_dev[MAX_DEV];

int64_t set_err(int64_t code, const char *msg) {
    put_err(msg);
    return code;
}

int cur_device(int64_t *rc) {
    int d = 0;
    hipError_t e = hipGetDevice(&d);
    if (e != hipSuccess) {
        *rc = det_fail_hip(e, "hipGetDevice");
        return -1;
    }
    if (d < 0 || d >= MAX_DEV) {
        *rc = set_err(DET_ERR_DEVICE, "device ordinal out of range");
        return -1;
    }
    return d;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Grow-only device buffer.  Growth waits for the device first, so a buffer
// still read by queued work is never freed underneath it.
int64_t ensure(void **buf, size_t *have, size_t need) {
    if (need <= *have) return 0;
    DET_HIP_CHECK(hipDeviceSynchronize());
    if (*buf) DET_HIP_CHECK(hipFree(*buf));
    *buf = nullptr;
    *have = 0;
    DET_HIP_CHECK(hipMalloc(buf, need));
    *have = need;
    return 0;
}

int64_t ensure_stream(DevState &d) {
    if (!d.stream) DET_HIP_CHECK(hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking));
    if (!d.ws_free) DET_HIP_CHECK(hipEventCreateWithFlags(&d.ws_free, hipEventDisableTiming));
    return 0;
}

// Release device d's state: wait until the library stream and the last
// workspace user are done, then free the staging buffer and the arena and
// destroy the stream and the event.  Caller holds ds.mu and has made d the
// current device.  Returns the first failure, but releases what it can.
int64_t release_device(DevState &ds) {
    int64_t rc = 0;
    auto step = [&](hipError_t e, const char *what) {
        if (e != hipSuccess && rc == 0) rc = det_fail_hip(e, what);
    };
    if (ds.stream) step(hipStreamSynchronize(ds.stream), "hipStreamSynchronize");
    if (ds.ws_free) step(hipEventSynchronize(ds.ws_free), "hipEventSynchronize");
    // The events and the stream go first: a recorded event keeps the copy
    // queued before it alive in the runtime, and with it the buffer that copy
    // wrote, whose memory would then come back only some time after hipFree.
    for (int i = 0; i < RING_SLOTS; ++i) {
        if (ds.ring_ev[i]) step(hipEventDestroy(ds.ring_ev[i]), "hipEventDestroy(ring)");
        ds.ring_ev[i] = nullptr;
        ds.ring_used[i] = false;
    }
    if (ds.ws_free) step(hipEventDestroy(ds.ws_free), "hipEventDestroy");
    if (ds.stream) step(hipStreamDestroy(ds.stream), "hipStreamDestroy");
    if (ds.io) step(hipFree(ds.io), "hipFree(staging)");
    if (ds.pin) step(hipHostFree(ds.pin), "hipHostFree(staging)");
    if (ds.ring) step(hipHostFree(ds.ring), "hipHostFree(ring)");
    ds.ring = ds.ring_dev = nullptr;
    ds.ring_next = 0;
    ds.ring_failed = false;
    if (ds.ws) step(hipFree(ds.ws), "hipFree(workspace)");
    ds.io = ds.ws = ds.pin = ds.pin_dev = nullptr;
    ds.pin_failed = false;
    ds.io_bytes = ds.ws_bytes = 0;
    ds.ws_free = nullptr;
    ds.stream = nullptr;
    return rc;
}

int64_t release_all() {
    int64_t rc = 0;
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    for (int d = 0; d < MAX_DEV; ++d) {
        DevState &ds = g_dev[d];
        std::lock_guard<std::mutex> lock(ds.mu);
        if (!ds.stream && !ds.ws_free && !ds.io && !ds.ws && !ds.pin && !ds.ring) continue;
        hipError_t e = hipSetDevice(d);
        int64_t r = e == hipSuccess ? release_device(ds) : det_fail_hip(e, "hipSetDevice");
        if (r && rc == 0) rc = r;
    }
    if (prev >= 0) (void)hipSetDevice(prev);
    return rc;
}


// ------------------------------------------------ host-pointer transfers
// Operands of a host-pointer call occupy one layout in the device staging
// buffer `io` (each at a 256-byte offset).  When the whole layout fits in
// PIN_BYTES it travels through a pinned host buffer of the same layout: the
// CPU copies the inputs into it, one kernel moves the input span into `io`
// (reading host memory over PCIe), and after the compute kernels another
// moves the output span back; the stream is synchronised and the CPU copies
// the outputs out.  A DMA copy costs about 10 us of latency here, from
// pageable and pinned memory alike, so a small call with three or four of
// them spent most of its time there; two kernels on the same stream cost a
// few microseconds.  In larger layouts each buffer of 1 MiB or more travels
// through the pinned ring below and smaller ones by hipMemcpyAsync on the
// caller's buffer; at about 3 MiB the pinned route and direct copies
// measured even.
constexpr size_t PIN_BYTES = 4u << 20;
// Outputs up to this size are written by the compute kernels straight into
// the pinned buffer (plain stores over PCIe), which saves the copy-back
// launch; larger ones come back through the copy kernel at full PCIe rate.
constexpr size_t OUT_DIRECT_BYTES = 256u << 10;
// Layouts up to this size whose kernel reads each input element only a few
// times (the tiny-shape GEMM kernels with at most 16 output tiles, the
// one-block dots) are read by the kernels straight from the pinned buffer
// too, which saves the copy-in launch as well (measured: 1-2 us at 16^3 -
// 64^3; at 128^3 the Q16 tiles' re-reads over PCIe cost more than the copy,
// and a one-block dot of 16384 terms, one workgroup reading 128 KiB over
// PCIe, took 33 instead of 24 us).  The GEMVs, the strict-f32 rows and the
// workspace-free FFTs, which read each input once, do so on the whole
// pinned route.
constexpr size_t IN_DIRECT_BYTES = 64u << 10;

struct HostIn {
    size_t off;
    const void *src;
    size_t bytes;
};
struct HostOut {
    size_t off;
    void *dst;
    size_t bytes;
};

__global__ __launch_bounds__(256) void copy16_kernel(uint4 *__restrict__ dst, const uint4 *__restrict__ src,
                                                     size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t copy16(void *dst, const void *src, size_t bytes, hipStream_t s) {
    const size_t n = (bytes + 15) / 16;
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, s, (uint4 *)dst,
                       (const uint4 *)src, n);
    return hipGetLastError();
}

// ---------------------------------------------- large transfers: the ring
// From the caller's pageable buffers the runtime's copies run at about
// 30 GB/s host to device and 18 GB/s back here, against 57 GB/s each way
// from pinned memory.  Buffers of at least RING_MIN bytes therefore travel
// in pieces through a ring of pinned chunks: the CPU copies a piece into
// its chunk while the DMA of the previous pieces runs (and, device to host,
// copies a landed piece out while later ones are in flight).  One CPU thread
// copies pageable memory at about 30 GB/s, so each piece's host copy is
// split over COPY_THREADS threads: 53-54 GB/s each way for a 1 GiB buffer.
constexpr size_t RING_MIN = 1u << 20;
// Pieces shorter than this move between a chunk and device memory by the
// copy kernel (a few microseconds of launch); longer ones by DMA, about 8%
// faster per byte from host memory but about 10 us of latency per copy.
constexpr size_t RING_DMA_MIN = 4u << 20;
using det::host::CopyPool;
CopyPool g_pool;

// True when this device's ring exists (allocated on the first large call and
// kept until teardown).  If the pinned allocation is refused, large calls
// copy the caller's buffers directly instead (the same results, the
// runtime's pageable rate).
bool ring_ready(DevState &ds) {
    if (ds.ring) return true;
    if (ds.ring_failed) return false;
    hipError_t e = hipHostMalloc((void **)&ds.ring, RING_SLOTS * RING_CHUNK, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void **)&ds.ring_dev, ds.ring, 0);
    for (int i = 0; i < RING_SLOTS && e == hipSuccess; ++i)
        e = hipEventCreateWithFlags(&ds.ring_ev[i], hipEventDisableTiming);
    if (e != hipSuccess) {
        for (int i = 0; i < RING_SLOTS; ++i) {
            if (ds.ring_ev[i]) (void)hipEventDestroy(ds.ring_ev[i]);
            ds.ring_ev[i] = nullptr;
        }
        if (ds.ring) (void)hipHostFree(ds.ring);
        ds.ring = nullptr;
        ds.ring_failed = true;
        (void)hipGetLastError();   // the refusal is handled: clear it
        return false;
    }
    return true;
}

// Piece length of a ring transfer of `bytes`: about a quarter of the
// buffer (so the copies of a mid-size buffer overlap too), 1 MiB to
// RING_CHUNK.
size_t ring_piece(size_t bytes) {
    const size_t q = ((bytes + 3) / 4 + ((1u << 20) - 1)) & ~(size_t)((1u << 20) - 1);
    return std::min(RING_CHUNK, q);
}

// Host -> device through the ring, asynchronous on s: each piece waits for
// its chunk's previous copy, is copied in by the CPU, and its DMA queued.
int64_t ring_h2d(DevState &ds, char *dst, const char *src, size_t bytes, hipStream_t s) {
    const size_t piece = ring_piece(bytes);
    for (size_t o = 0; o < bytes; o += piece) {
        const size_t n = std::min(piece, bytes - o);
        const unsigned sl = ds.ring_next++ % RING_SLOTS;
        char *chunk = ds.ring + (size_t)sl * RING_CHUNK;
        if (ds.ring_used[sl]) DET_HIP_CHECK(hipEventSynchronize(ds.ring_ev[sl]));
        g_pool.copy(chunk, src + o, n);
        if (n < RING_DMA_MIN) DET_HIP_CHECK(copy16(dst + o, ds.ring_dev + (size_t)sl * RING_CHUNK, n, s));
        else DET_HIP_CHECK(hipMemcpyAsync(dst + o, chunk, n, hipMemcpyHostToDevice, s));
        DET_HIP_CHECK(hipEventRecord(ds.ring_ev[sl], s));
        ds.ring_used[sl] = true;
    }
    return 0;
}

// Device -> host through the ring, after the work queued on s: up to
// RING_SLOTS pieces in flight; each landed piece is copied out by the CPU
// and its chunk refilled with the next piece.  A chunk's earlier user is a
// copy queued on s before (ordered by the stream) or a piece whose host
// copy has finished, so no piece waits for anything but its own DMA.
int64_t ring_d2h(DevState &ds, char *dst, const char *src, size_t bytes, hipStream_t s) {
    const size_t piece = ring_piece(bytes), np = (bytes + piece - 1) / piece;
    const unsigned first = ds.ring_next;
    ds.ring_next += (unsigned)np;
    auto issue = [&](size_t i) -> int64_t {
        const unsigned sl = (first + (unsigned)i) % RING_SLOTS;
        const size_t o = i * piece;
        const size_t n = std::min(piece, bytes - o);
        if (n < RING_DMA_MIN) DET_HIP_CHECK(copy16(ds.ring_dev + (size_t)sl * RING_CHUNK, src + o, n, s));
        else DET_HIP_CHECK(hipMemcpyAsync(ds.ring + (size_t)sl * RING_CHUNK, src + o, n, hipMemcpyDeviceToHost, s));
        DET_HIP_CHECK(hipEventRecord(ds.ring_ev[sl], s));
        ds.ring_used[sl] = true;
        return 0;
    };
    int64_t rc = 0;
    for (size_t i = 0; i < np && i < (size_t)RING_SLOTS; ++i)
        if ((rc = issue(i))) return rc;
    for (size_t i = 0; i < np; ++i) {
        const unsigned sl = (first + (unsigned)i) % RING_SLOTS;
        DET_HIP_CHECK(hipEventSynchronize(ds.ring_ev[sl]));
        const size_t o = i * piece;
        g_pool.copy(dst + o, ds.ring + (size_t)sl * RING_CHUNK, std::min(piece, bytes - o));
        if (i + RING_SLOTS < np && (rc = issue(i + RING_SLOTS))) return rc;
    }
    return 0;
}

// True when a layout of `span` bytes takes the pinned route (the buffer is
// allocated on the first such call and kept until teardown).  If the pinned
// allocation is refused, this device's small calls copy directly instead
// (the same results, the DMA route's latency).
bool pinned_route(DevState &ds, size_t span) {
    if (span > PIN_BYTES || ds.pin_failed) return false;
    if (!ds.pin) {
        hipError_t e = hipHostMalloc(&ds.pin, PIN_BYTES, hipHostMallocDefault);
        if (e == hipSuccess) e = hipHostGetDevicePointer(&ds.pin_dev, ds.pin, 0);
        if (e != hipSuccess) {
            if (ds.pin) (void)hipHostFree(ds.pin);
            ds.pin = ds.pin_dev = nullptr;
            ds.pin_failed = true;
            (void)hipGetLastError();   // the refusal is handled: clear it
            return false;
        }
    }
    return true;
}

// Inputs into io (asynchronous on s), or only into the pinned buffer when
// the kernels read them there (`direct`).
int64_t put_inputs(DevState &ds, bool pinned, const HostIn *in, int n_in, hipStream_t s, bool direct = false) {
    char *io = (char *)ds.io;
    if (!pinned) {
        int64_t rc = 0;
        for (int i = 0; i < n_in; ++i) {
            if (in[i].bytes >= RING_MIN && ring_ready(ds)) {
                if ((rc = ring_h2d(ds, io + in[i].off, (const char *)in[i].src, in[i].bytes, s))) return rc;
            } else if (in[i].bytes) {
                DET_HIP_CHECK(hipMemcpyAsync(io + in[i].off, in[i].src, in[i].bytes, hipMemcpyHostToDevice, s));
            }
        }
        return 0;
    }
    size_t end = 0, total = 0;
    for (int i = 0; i < n_in; ++i) total += in[i].bytes;
    // large layouts: each input's copy kernel is queued as soon as its host
    // copy is done, so it runs while the CPU copies the next input
    const bool staged = !direct && total >= (512u << 10);
    for (int i = 0; i < n_in; ++i) {
        if (in[i].bytes) g_pool.copy((char *)ds.pin + in[i].off, in[i].src, in[i].bytes);
        if (staged && in[i].bytes)
            DET_HIP_CHECK(copy16(io + in[i].off, (char *)ds.pin_dev + in[i].off, in[i].bytes, s));
        if (in[i].off + in[i].bytes > end) end = in[i].off + in[i].bytes;
    }
    if (!direct && !staged) DET_HIP_CHECK(copy16(io, ds.pin_dev, end, s));
    return 0;
}

// Where a compute kernel writes an output of `bytes` at layout offset `off`:
// the pinned buffer itself for small outputs on the pinned route (`direct`),
// else the device staging buffer.
void *out_ptr(DevState &ds, bool pinned, size_t off, size_t bytes, bool *direct) {
    *direct = pinned && bytes <= OUT_DIRECT_BYTES;
    return (*direct ? (char *)ds.pin_dev : (char *)ds.io) + off;
}

// Outputs out of io (or already in the pinned buffer when `direct`), then
// wait for the stream.  The outputs' offsets are 256-byte aligned, so the
// span copied back starts on a 16-byte boundary.
int64_t get_outputs(DevState &ds, bool pinned, const HostOut *out, int n_out, hipStream_t s, bool direct = false) {
    char *io = (char *)ds.io;
    if (!pinned) {
        int64_t rc = 0;
        for (int i = 0; i < n_out; ++i) {
            if (out[i].bytes >= RING_MIN && ring_ready(ds)) {
                if ((rc = ring_d2h(ds, (char *)out[i].dst, io + out[i].off, out[i].bytes, s))) return rc;
            } else if (out[i].bytes) {
                DET_HIP_CHECK(hipMemcpyAsync(out[i].dst, io + out[i].off, out[i].bytes, hipMemcpyDeviceToHost, s));
            }
        }
        DET_HIP_CHECK(hipStreamSynchronize(s));
        return 0;
    }
    size_t lo = (size_t)-1, hi = 0;
    for (int i = 0; i < n_out; ++i) {
        if (out[i].off < lo) lo = out[i].off;
        if (out[i].off + out[i].bytes > hi) hi = out[i].off + out[i].bytes;
    }
    if (hi > lo && !direct) DET_HIP_CHECK(copy16((char *)ds.pin_dev + lo, io + lo, hi - lo, s));
    DET_HIP_CHECK(hipStreamSynchronize(s));
    for (int i = 0; i < n_out; ++i)
        if (out[i].bytes) g_pool.copy(out[i].dst, (const char *)ds.pin + out[i].off, out[i].bytes);
    return 0;
}

bool bad_dims(int64_t m, int64_t k, int64_t n) {
    return m < 0 || k < 0 || n < 0 || m > DIM_MAX || k > DIM_MAX || n > DIM_MAX;
}

// Zero an int32 buffer (used for K == 0: the exact sum over no terms).
__global__ void fill_zero_i32(int32_t *p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

hipError_t zero_i32(int32_t *p, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_i32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------- device ops
enum class Op { I8, I16, Q16, Q16_BT };

size_t elem_bytes(Op op) { return op == Op::I8 ? 1 : op == Op::I16 ? 2 : 4; }

// Launch one GEMM on device pointers.  `ws` must hold the limb workspace for
// I16 / Q16 (ignored for I8).
int64_t gemm_dev(Op op, const void *A, const void *B, void *C, int64_t m, int64_t k, int64_t n, void *ws,
                 hipStream_t s) {
    const int M = (int)m, N = (int)n, K = (int)k;
    if (K == 0) DET_HIP_CHECK(zero_i32((int32_t *)C, (size_t)m * n, s));
    else if (op == Op::I8)
        DET_HIP_CHECK(det::launch_gemm_i8((const int8_t *)A, (const int8_t *)B, (int32_t *)C, M, N, K, ws, s));
    else if (op == Op::I16)
        DET_HIP_CHECK(det::launch_gemm_i16((const int16_t *)A, (const int16_t *)B, (int32_t *)C, M, N, K, ws, s));
    else
        DET_HIP_CHECK(det::launch_gemm_q16((const int32_t *)A, (const int32_t *)B, (int32_t *)C, M, N, K,
                                           op == Op::Q16_BT, ws, s));
    return 0;
}

bool aligned16(const void *a, const void *b) { return (((uintptr_t)a | (uintptr_t)b) & 15) == 0; }

// Workspace bytes of one GEMM.  int8 needs one only for operands off the
// 16-byte grid, or small grids the edge kernel would underfill (repacked
// into padded panels), which depends on the operand addresses; NULL operands
// are taken as aligned.
size_t ws_need(Op op, int64_t m, int64_t k, int64_t n, const void *A = nullptr, const void *B = nullptr) {
    if (k == 0) return 0;
    if (op == Op::I8) return det::i8_workspace_bytes((int)m, (int)n, (int)k, aligned16(A, B));
    return op == Op::I16 ? det::i16_workspace_bytes((int)m, (int)n, (int)k)
                         : det::q16_workspace_bytes((int)m, (int)n, (int)k);
}

// Device-pointer GEMM using the library workspace arena (ordered after the
// arena's previous user through the ws_free event).
int64_t gemm_dev_arena(Op op, const void *A, const void *B, void *C, int64_t m, int64_t k, int64_t n,
                       hipStream_t s) {
    if (bad_dims(m, k, n)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0 || n == 0) return 0;
    if (!A || !B || !C) return set_err(DET_ERR_ARG, "null device pointer");
    const size_t need = ws_need(op, m, k, n, A, B);
    if (need == 0) return gemm_dev(op, A, B, C, m, k, n, nullptr, s);
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    if ((rc = ensure(&ds.ws, &ds.ws_bytes, need))) return rc;
    DET_HIP_CHECK(hipStreamWaitEvent(s, ds.ws_free, 0));
    if ((rc = gemm_dev(op, A, B, C, m, k, n, ds.ws, s))) return rc;
    DET_HIP_CHECK(hipEventRecord(ds.ws_free, s));
    return 0;
}

// Host-pointer GEMM: stage, launch, copy back, wait.
int64_t gemm_host(Op op, int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    if (bad_dims(m, k, n)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0 || n == 0) return 0;
    if (!c || ((!a || !b) && k > 0)) return 0;   // Track A: NULL -> 0, nothing written
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    const size_t eb = elem_bytes(op);
    const size_t bytes_a = (size_t)m * k * eb, bytes_b = (size_t)k * n * eb, bytes_c = (size_t)m * n * 4;
    const size_t off_b = align256(bytes_a), off_c = off_b + align256(bytes_b);
    const size_t span = off_c + align256(bytes_c), need = ws_need(op, m, k, n);
    if ((rc = ensure(&ds.io, &ds.io_bytes, span))) return rc;
    if ((rc = ensure(&ds.ws, &ds.ws_bytes, need))) return rc;
    const bool pinned = pinned_route(ds, span);
    hipStream_t s = ds.stream;
    // the tiny-shape kernels over at most 16 output tiles read the inputs
    // from the pinned buffer itself when the layout is small
    const int M = (int)m, N = (int)n, K = (int)k;
    const bool tiny = op == Op::I8 ? det::i8_small(M, N, K) : op == Op::I16 ? det::i16_small(M, N, K)
                                                                            : det::q16_small(M, N, K);
    const bool in_direct = pinned && tiny && span <= IN_DIRECT_BYTES && ((m + 15) / 16) * ((n + 15) / 16) <= 16;
    char *io = in_direct ? (char *)ds.pin_dev : (char *)ds.io;
    const HostIn in[2] = {{0, (const void *)a, bytes_a}, {off_b, (const void *)b, bytes_b}};
    if ((rc = put_inputs(ds, pinned, in, 2, s, in_direct))) return rc;
    // the workspace arena is shared with the device-pointer entry points:
    // start after its last user, and mark this stream as its next one
    if (need) DET_HIP_CHECK(hipStreamWaitEvent(s, ds.ws_free, 0));
    bool direct = false;
    void *dc = out_ptr(ds, pinned, off_c, bytes_c, &direct);
    if ((rc = gemm_dev(op, io, io + off_b, dc, m, k, n, need ? ds.ws : nullptr, s))) return rc;
    if (need) DET_HIP_CHECK(hipEventRecord(ds.ws_free, s));
    const HostOut out[1] = {{off_c, (void *)c, bytes_c}};
    return get_outputs(ds, pinned, out, 1, s, direct);
}

// Q16 GEMV over nb vectors on device pointers: groups of up to 8 vectors go
// to the MFMA kernel when the shape allows it (and nb >= 2), the rest to the
// one-vector VALU kernel.  `ws` must hold gemv8_workspace_bytes(K) when
// gemv_ws_need() is non-zero.
size_t gemv_ws_need(const int32_t *W, const int32_t *X, int64_t m, int64_t k, int64_t nb) {
    if (nb < 2 || k == 0 || !det::gemv8_eligible(W, X, (int)m, (int)k)) return 0;
    return det::gemv8_workspace_bytes((int)k);
}

hipError_t gemv_q16_any(const int32_t *W, const int32_t *X, int32_t *Y, int64_t m, int64_t k, int64_t nb, void *ws,
                        hipStream_t s) {
    const int M = (int)m, K = (int)k;
    if (K == 0) return zero_i32(Y, (size_t)m * nb, s);
    if (!ws || nb < 2) return det::launch_gemv_q16(W, X, Y, M, K, (int)nb, s);
    for (int64_t b = 0; b < nb; b += 8) {
        const int g = (int)(nb - b < 8 ? nb - b : 8);
        hipError_t e = g >= 2 ? det::launch_gemv_q16_mfma(W, X + b * k, Y + b * m, M, K, g, ws, s)
                              : det::launch_gemv_q16(W, X + b * k, Y + b * m, M, K, g, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Host-pointer GEMV family (Q16 batched, int16).
int64_t gemv_host(bool q16, int64_t w, int64_t x, int64_t y, int64_t m, int64_t k, int64_t nb) {
    if (bad_dims(m, k, nb)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0 || nb == 0) return 0;
    if (!y || ((!w || !x) && k > 0)) return 0;
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    const size_t eb = q16 ? 4 : 2;
    const size_t bytes_w = (size_t)m * k * eb, bytes_x = (size_t)nb * k * eb, bytes_y = (size_t)nb * m * 4;
    const size_t off_x = align256(bytes_w), off_y = off_x + align256(bytes_x);
    const size_t span = off_y + align256(bytes_y);
    if ((rc = ensure(&ds.io, &ds.io_bytes, span))) return rc;
    const bool pinned = pinned_route(ds, span);
    // W is read once and x once per row group: on the pinned route the
    // kernels read both straight from the pinned buffer at every size
    // (measured against copying them in first: mmi16 512^2 36.9 -> 32.0 us,
    // gemvq 1000^2 145 -> 120 us)
    const bool in_direct = pinned;
    char *io = in_direct ? (char *)ds.pin_dev : (char *)ds.io;
    hipStream_t s = ds.stream;
    const HostIn in[2] = {{0, (const void *)w, bytes_w}, {off_x, (const void *)x, bytes_x}};
    if ((rc = put_inputs(ds, pinned, in, 2, s, in_direct))) return rc;
    bool direct = false;
    int32_t *dy = (int32_t *)out_ptr(ds, pinned, off_y, bytes_y, &direct);
    if (k == 0) DET_HIP_CHECK(zero_i32(dy, (size_t)nb * m, s));
    else if (q16) {
        const int32_t *dW = (const int32_t *)io, *dX = (const int32_t *)(io + off_x);
        const size_t need = gemv_ws_need(dW, dX, m, k, nb);
        if ((rc = ensure(&ds.ws, &ds.ws_bytes, need))) return rc;
        // the workspace arena is shared with the device-pointer entry points
        // (other streams): start after its last user, then mark this stream
        if (need) DET_HIP_CHECK(hipStreamWaitEvent(s, ds.ws_free, 0));
        DET_HIP_CHECK(gemv_q16_any(dW, dX, dy, m, k, nb, need ? ds.ws : nullptr, s));
        if (need) DET_HIP_CHECK(hipEventRecord(ds.ws_free, s));
    } else
        DET_HIP_CHECK(det::launch_gemv_i16((const int16_t *)io, (const int16_t *)(io + off_x), dy, (int)m, (int)k, s));
    const HostOut out[1] = {{off_y, (void *)y, bytes_y}};
    return get_outputs(ds, pinned, out, 1, s, direct);
}

// Host-pointer vector reductions: (int64)(int32)sum; len <= 0 or a NULL
// pointer returns 0 (the reference's Track A convention).
int64_t dot_host(int op, int64_t a, int64_t b, int64_t len) {
    if (len <= 0 || !a || !b) return 0;
    if (len >= (1LL << 31)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    const size_t eb = op == det::DOT_I16 ? 2 : 4, bytes = (size_t)len * eb;
    const size_t off_b = align256(bytes), off_o = off_b + align256(bytes);
    const size_t span = off_o + 256;
    if ((rc = ensure(&ds.io, &ds.io_bytes, span))) return rc;
    const bool pinned = pinned_route(ds, span);
    // a dot one block covers stores its sum with a plain store: straight into
    // the pinned buffer, its inputs read from there too when they are small
    const bool single = pinned && det::dot_single_block(len);
    const bool in_direct = single && span <= IN_DIRECT_BYTES;
    char *io = in_direct ? (char *)ds.pin_dev : (char *)ds.io;
    hipStream_t s = ds.stream;
    const HostIn in[2] = {{0, (const void *)a, bytes}, {off_b, (const void *)b, bytes}};
    if ((rc = put_inputs(ds, pinned, in, 2, s, in_direct))) return rc;
    uint32_t *dout = (uint32_t *)((single ? (char *)ds.pin_dev : (char *)ds.io) + off_o);
    DET_HIP_CHECK(det::launch_dot(op, io, io + off_b, len, dout, s));
    uint32_t res = 0;
    const HostOut out[1] = {{off_o, &res, 4}};
    if ((rc = get_outputs(ds, pinned, out, 1, s, single))) return rc;
    return (int64_t)(int32_t)res;
}

// Host-pointer strict-FP f32 rows: y[r] = metric met of (W row r, x).
// rows, cols > 0.
int64_t f32_rows_host(const float *w, const float *x, float *y, int64_t rows, int64_t cols, int met) {
    if (rows >= (1LL << 31) || cols >= (1LL << 31)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    const size_t bytes_w = (size_t)rows * cols * 4, bytes_x = (size_t)cols * 4, bytes_y = (size_t)rows * 4;
    const size_t off_x = align256(bytes_w), off_y = off_x + align256(bytes_x);
    const size_t span = off_y + align256(bytes_y);
    if ((rc = ensure(&ds.io, &ds.io_bytes, span))) return rc;
    const bool pinned = pinned_route(ds, span);
    // W read once: the kernel reads the inputs straight from the pinned
    // buffer on the whole pinned route (512^2 56-61 -> 42-51 us)
    char *io = pinned ? (char *)ds.pin_dev : (char *)ds.io;
    hipStream_t s = ds.stream;
    const HostIn in[2] = {{0, w, bytes_w}, {off_x, x, bytes_x}};
    if ((rc = put_inputs(ds, pinned, in, 2, s, pinned))) return rc;
    bool direct = false;
    float *dy = (float *)out_ptr(ds, pinned, off_y, bytes_y, &direct);
    DET_HIP_CHECK(det::launch_rows_f32((const float *)io, (const float *)(io + off_x), dy, rows, cols, met, s));
    const HostOut out[1] = {{off_y, y, bytes_y}};
    return get_outputs(ds, pinned, out, 1, s, direct);
}

// The reference's packing of an f32 result: its bits, zero-extended to int64.
int64_t pack_f32(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return (int64_t)(uint64_t)b;
}

// The packed f32 return cannot carry an error code (a failure returns the
// bits of +0.0f), so the error text is cleared on entry: after the call an
// empty det_last_error() means success.
int64_t dot_f32_host(int64_t a, int64_t b, int64_t len, int met = det::F32_DOT) {
    g_err[0] = 0;
    if (len <= 0 || !a || !b) return pack_f32(0.0f);
    float out = 0.0f;
    if (f32_rows_host((const float *)(intptr_t)a, (const float *)(intptr_t)b, &out, 1, len, met) != 0) return 0;
    return pack_f32(out);
}


// ---------------------------------------------------------------- Q16 FFT
// Argument check shared by the FFT entry points: 1 = nothing to transform
// (n == 0 or batch == 0: the reference's loops run zero times), 0 = run,
// negative = error.  n must be 2^logn with logn in [0, 30] (the reference
// kernel indexes out of its buffers otherwise), and batch * n <= 2^31.
int64_t fft_check(int64_t logn, int64_t n, int64_t batch) {
    if (batch < 0 || n < 0) return set_err(DET_ERR_ARG, "fft: negative size");
    if (n == 0 || batch == 0) return 1;
    if (logn < 0 || logn > 30 || n != ((int64_t)1 << logn))
        return set_err(DET_ERR_ARG, "fft: n must equal 2^logn with logn in [0, 30]");
    // 2^31 points = 32 GiB of re + im; keeps every FFT grid far below 2^32 work-items
    if (batch > ((int64_t)1 << 31) / n) return set_err(DET_ERR_ARG, "fft: batch * n exceeds 2^31 points");
    return 0;
}

// Device-pointer FFT on stream s; the n >= 4096 path borrows the workspace
// arena (ordered after its previous user).  Call with ds.mu NOT held.
int64_t fft_dev_run(const int64_t *sre, const int64_t *sim, int64_t *dre, int64_t *dim, const int64_t *tw, int logn,
                    int64_t batch, hipStream_t s) {
    const size_t need = det::fft_workspace_bytes(logn, batch);
    if (need == 0) {
        DET_HIP_CHECK(det::launch_fft_q16(sre, sim, dre, dim, tw, logn, batch, nullptr, s));
        return 0;
    }
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    if ((rc = ensure(&ds.ws, &ds.ws_bytes, need))) return rc;
    DET_HIP_CHECK(hipStreamWaitEvent(s, ds.ws_free, 0));
    DET_HIP_CHECK(det::launch_fft_q16(sre, sim, dre, dim, tw, logn, batch, ds.ws, s));
    DET_HIP_CHECK(hipEventRecord(ds.ws_free, s));
    return 0;
}

// Host-pointer FFT: batch transforms of n points at re / im (in place),
// twiddle table tw (n int64 = n / 2 (wr, wi) pairs; unused for n < 4).
int64_t fft_host(int64_t re, int64_t im, int64_t tw, int64_t logn, int64_t n, int64_t batch) {
    int64_t rc = fft_check(logn, n, batch);
    if (rc) return rc > 0 ? 0 : rc;
    if (!re || !im || (!tw && n >= 4)) return set_err(DET_ERR_ARG, "fft: null pointer");
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    const size_t bytes = (size_t)batch * n * 8, bytes_tw = n >= 4 ? (size_t)n * 8 : 0;
    const size_t off_im = align256(bytes), off_tw = off_im + align256(bytes);
    const size_t span = off_tw + align256(bytes_tw) + 256;
    if ((rc = ensure(&ds.io, &ds.io_bytes, span))) return rc;
    const size_t need = det::fft_workspace_bytes((int)logn, batch);
    if ((rc = ensure(&ds.ws, &ds.ws_bytes, need))) return rc;
    const bool pinned = pinned_route(ds, span);
    // a few small transforms (no workspace: one read and one write per
    // point, in place) run on the pinned buffer itself: no copy launches
    // the LDS kernels read each point once and write it once: in and out
    // through the pinned buffer itself on the whole pinned route (batch 64
    // of 256 points 41.5 -> 35.5 us)
    const bool direct = pinned && need == 0;
    char *io = direct ? (char *)ds.pin_dev : (char *)ds.io;
    hipStream_t s = ds.stream;
    const HostIn in[3] = {{0, (const void *)re, bytes}, {off_im, (const void *)im, bytes},
                          {off_tw, (const void *)tw, bytes_tw}};
    if ((rc = put_inputs(ds, pinned, in, 3, s, direct))) return rc;
    if (need) DET_HIP_CHECK(hipStreamWaitEvent(s, ds.ws_free, 0));
    int64_t *dre = (int64_t *)io, *dim = (int64_t *)(io + off_im);
    DET_HIP_CHECK(det::launch_fft_q16(dre, dim, dre, dim, (const int64_t *)(io + off_tw), (int)logn, batch,
                                      need ? ds.ws : nullptr, s));
    if (need) DET_HIP_CHECK(hipEventRecord(ds.ws_free, s));
    const HostOut out[2] = {{0, (void *)re, bytes}, {off_im, (void *)im, bytes}};
    return get_outputs(ds, pinned, out, 2, s, direct);
}

}  // namespace

extern "C" int64_t det_fail_hip(hipError_t e, const char *what) {
    put_err(what, hipGetErrorString(e));
    return DET_ERR_HIP;
}

extern "C" int64_t det_fail(int64_t code, const char *msg) { return set_err(code, msg); }

// ====================================================================== layer 1
extern "C" {

int64_t __mind_blas_matmul_mm_i8_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::I8, a, b, c, m, k, n);
}
int64_t __mind_blas_matmul_mm_i8_mt_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::I8, a, b, c, m, k, n);
}
int64_t __mind_blas_matmul_mm_q16_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::Q16, a, b, c, m, k, n);
}
int64_t __mind_blas_matmul_mm_q16_mt_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::Q16, a, b, c, m, k, n);
}
int64_t __mind_blas_gemv_q16_mt(int64_t w, int64_t x, int64_t y, int64_t m, int64_t k) {
    return gemv_host(true, w, x, y, m, k, 1);
}
int64_t __mind_blas_matmul_rmajor_q16_v(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    return gemv_host(true, w, x, y, rows, cols, 1);
}
int64_t __mind_blas_matmul_rmajor_i16_v(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    return gemv_host(false, w, x, y, rows, cols, 1);
}
int64_t __mind_blas_dot_q16(int64_t a, int64_t b, int64_t len) { return dot_host(det::DOT_Q16, a, b, len); }
int64_t __mind_blas_dot_q16_v(int64_t a, int64_t b, int64_t len) { return dot_host(det::DOT_Q16, a, b, len); }
int64_t __mind_blas_dot_l1_q16(int64_t a, int64_t b, int64_t len) { return dot_host(det::DOT_L1, a, b, len); }
int64_t __mind_blas_dot_l1_q16_v(int64_t a, int64_t b, int64_t len) { return dot_host(det::DOT_L1, a, b, len); }
int64_t __mind_blas_dot_i16_v(int64_t a, int64_t b, int64_t len) { return dot_host(det::DOT_I16, a, b, len); }
int64_t __mind_blas_dot_f32(int64_t a, int64_t b, int64_t len) { return dot_f32_host(a, b, len); }
int64_t __mind_blas_dot_f32_v(int64_t a, int64_t b, int64_t len) { return dot_f32_host(a, b, len); }
int64_t __mind_blas_dot_l1_f32(int64_t a, int64_t b, int64_t len) { return dot_f32_host(a, b, len, det::F32_L1); }
int64_t __mind_blas_dot_l1_f32_v(int64_t a, int64_t b, int64_t len) { return dot_f32_host(a, b, len, det::F32_L1); }
int64_t __mind_blas_dot_linf_f32(int64_t a, int64_t b, int64_t len) {
    return dot_f32_host(a, b, len, det::F32_LINF);
}
int64_t __mind_blas_dot_linf_f32_v(int64_t a, int64_t b, int64_t len) {
    return dot_f32_host(a, b, len, det::F32_LINF_V);
}
int64_t __mind_blas_matmul_rmajor_f32(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    if (!w || !x || !y) return -1;
    if (rows <= 0 || cols <= 0) return 0;
    return f32_rows_host((const float *)(intptr_t)w, (const float *)(intptr_t)x, (float *)(intptr_t)y, rows, cols,
                         det::F32_DOT);
}
int64_t __mind_blas_matmul_rmajor_f32_v(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    if (!w || !x || !y || rows <= 0 || cols <= 0) return 0;
    return f32_rows_host((const float *)(intptr_t)w, (const float *)(intptr_t)x, (float *)(intptr_t)y, rows, cols,
                         det::F32_DOT);
}

// ====================================================================== layer 2
int64_t gemmi8(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return __mind_blas_matmul_mm_i8_v(a, b, c, m, k, n);
}
int64_t gemmi8mt(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return __mind_blas_matmul_mm_i8_mt_v(a, b, c, m, k, n);
}
int64_t gemmqmm(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return __mind_blas_matmul_mm_q16_v(a, b, c, m, k, n);
}
int64_t gemmq(int64_t a, int64_t bt, int64_t c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::Q16_BT, a, bt, c, m, k, n);
}
int64_t mmq(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    return __mind_blas_matmul_rmajor_q16_v(w, x, y, rows, cols);
}
int64_t mmi16(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    return __mind_blas_matmul_rmajor_i16_v(w, x, y, rows, cols);
}
int64_t gemvq(int64_t catalog, int64_t query, int64_t scores, int64_t m, int64_t k) {
    return __mind_blas_gemv_q16_mt(catalog, query, scores, m, k);
}
int64_t dotq(int64_t a, int64_t b, int64_t n) { return __mind_blas_dot_q16_v(a, b, n); }
int64_t dotl1q(int64_t a, int64_t b, int64_t n) { return __mind_blas_dot_l1_q16_v(a, b, n); }
int64_t doti16(int64_t a, int64_t b, int64_t n) { return __mind_blas_dot_i16_v(a, b, n); }
int64_t dotf32(int64_t a, int64_t b, int64_t n) { return __mind_blas_dot_f32_v(a, b, n); }
int64_t fft256(int64_t re, int64_t im, int64_t tw, int64_t logn, int64_t n) {
    return fft_host(re, im, tw, logn, n, 1);
}
int64_t mmf32(int64_t w, int64_t x, int64_t y, int64_t rows, int64_t cols) {
    return __mind_blas_matmul_rmajor_f32_v(w, x, y, rows, cols);
}

// ====================================================================== layer 3
int64_t det_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::I8, (int64_t)a, (int64_t)b, (int64_t)c, m, k, n);
}
int64_t det_matmul_i16(const int16_t *a, const int16_t *b, int32_t *c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::I16, (int64_t)a, (int64_t)b, (int64_t)c, m, k, n);
}
int64_t det_matmul_q16(const int32_t *a, const int32_t *b, int32_t *c, int64_t m, int64_t k, int64_t n) {
    return gemm_host(Op::Q16, (int64_t)a, (int64_t)b, (int64_t)c, m, k, n);
}
int64_t det_gemv_q16(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k) {
    return gemv_host(true, (int64_t)w, (int64_t)x, (int64_t)y, m, k, 1);
}
int64_t det_gemv_q16_batched(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k, int64_t nb) {
    return gemv_host(true, (int64_t)w, (int64_t)x, (int64_t)y, m, k, nb);
}
int64_t det_gemv_i16(const int16_t *w, const int16_t *x, int32_t *y, int64_t m, int64_t k) {
    return gemv_host(false, (int64_t)w, (int64_t)x, (int64_t)y, m, k, 1);
}
int64_t det_dot_q16(const int32_t *a, const int32_t *b, int64_t len) {
    return dot_host(det::DOT_Q16, (int64_t)(intptr_t)a, (int64_t)(intptr_t)b, len);
}
int64_t det_dot_l1_q16(const int32_t *a, const int32_t *b, int64_t len) {
    return dot_host(det::DOT_L1, (int64_t)(intptr_t)a, (int64_t)(intptr_t)b, len);
}
int64_t det_dot_i16(const int16_t *a, const int16_t *b, int64_t len) {
    return dot_host(det::DOT_I16, (int64_t)(intptr_t)a, (int64_t)(intptr_t)b, len);
}
int64_t det_dot_f32(const float *a, const float *b, int64_t len, float *out) {
    if (!out) return set_err(DET_ERR_ARG, "null output pointer");
    if (len <= 0 || !a || !b) {
        *out = 0.0f;
        return 0;
    }
    return f32_rows_host(a, b, out, 1, len, det::F32_DOT);
}
int64_t det_matmul_rmajor_f32(const float *w, const float *x, float *y, int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (rows == 0 || cols == 0 || !w || !x || !y) return 0;
    return f32_rows_host(w, x, y, rows, cols, det::F32_DOT);
}

int64_t det_matmul_i8_dev(const int8_t *a, const int8_t *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                          void *stream) {
    return gemm_dev_arena(Op::I8, a, b, c, m, k, n, (hipStream_t)stream);
}
int64_t det_matmul_i16_dev(const int16_t *a, const int16_t *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                           void *stream) {
    return gemm_dev_arena(Op::I16, a, b, c, m, k, n, (hipStream_t)stream);
}
int64_t det_matmul_q16_dev(const int32_t *a, const int32_t *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                           void *stream) {
    return gemm_dev_arena(Op::Q16, a, b, c, m, k, n, (hipStream_t)stream);
}

int64_t det_workspace_bytes(int64_t op, int64_t m, int64_t k, int64_t n) {
    if (bad_dims(m, k, n) || m == 0 || n == 0) return 0;
    if (op == DET_OP_I8) return (int64_t)ws_need(Op::I8, m, k, n);
    if (op == DET_OP_I16) return (int64_t)ws_need(Op::I16, m, k, n);
    if (op == DET_OP_Q16) return (int64_t)ws_need(Op::Q16, m, k, n);
    return 0;
}

int64_t det_matmul_ws_dev(int64_t op, const void *a, const void *b, int32_t *c, int64_t m, int64_t k, int64_t n,
                          void *ws, int64_t ws_bytes, void *stream) {
    if (bad_dims(m, k, n)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0 || n == 0) return 0;
    if (!a || !b || !c) return set_err(DET_ERR_ARG, "null device pointer");
    Op o;
    if (op == DET_OP_I8) o = Op::I8;
    else if (op == DET_OP_I16) o = Op::I16;
    else if (op == DET_OP_Q16) o = Op::Q16;
    else return set_err(DET_ERR_ARG, "unknown op");
    const size_t need = ws_need(o, m, k, n, a, b);
    const bool enough = ws_bytes >= 0 && (size_t)ws_bytes >= need && (need == 0 || ws);
    // int8 runs without a workspace too (operands off the 16-byte grid then
    // take the byte-load kernel); the limb GEMMs cannot
    if (!enough && o != Op::I8) return set_err(DET_ERR_ARG, "workspace too small (see det_workspace_bytes)");
    return gemm_dev(o, a, b, c, m, k, n, enough ? ws : nullptr, (hipStream_t)stream);
}

// The batched GEMV's workspace (the query vectors' MFMA operands), assuming
// aligned operands: 0 when no group of vectors takes the MFMA kernel.
int64_t det_gemv_workspace_bytes(int64_t m, int64_t k, int64_t nb) {
    if (bad_dims(m, k, nb) || m == 0 || nb == 0) return 0;
    return (int64_t)gemv_ws_need(nullptr, nullptr, m, k, nb);
}

// det_gemv_q16_dev with the caller's workspace: no arena, so no allocation
// and no event ordering; a short or missing workspace takes the VALU kernel.
int64_t det_gemv_q16_ws_dev(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k, int64_t nb,
                            void *ws, int64_t ws_bytes, void *stream) {
    if (bad_dims(m, k, nb)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0 || nb == 0) return 0;
    if (!y || ((!w || !x) && k > 0)) return set_err(DET_ERR_ARG, "null device pointer");
    const size_t need = gemv_ws_need(w, x, m, k, nb);
    const bool enough = need && ws && ws_bytes >= 0 && (size_t)ws_bytes >= need;
    DET_HIP_CHECK(gemv_q16_any(w, x, y, m, k, nb, enough ? ws : nullptr, (hipStream_t)stream));
    return 0;
}

int64_t det_gemv_q16_dev(const int32_t *w, const int32_t *x, int32_t *y, int64_t m, int64_t k, int64_t nb,
                         void *stream) {
    if (bad_dims(m, k, nb)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0 || nb == 0) return 0;
    if (!y || ((!w || !x) && k > 0)) return set_err(DET_ERR_ARG, "null device pointer");
    hipStream_t s = (hipStream_t)stream;
    const size_t need = gemv_ws_need(w, x, m, k, nb);
    if (need == 0) {
        DET_HIP_CHECK(gemv_q16_any(w, x, y, m, k, nb, nullptr, s));
        return 0;
    }
    int64_t rc = 0;
    const int d = cur_device(&rc);
    if (d < 0) return rc;
    DevState &ds = g_dev[d];
    std::lock_guard<std::mutex> lock(ds.mu);
    if ((rc = ensure_stream(ds))) return rc;
    if ((rc = ensure(&ds.ws, &ds.ws_bytes, need))) return rc;
    DET_HIP_CHECK(hipStreamWaitEvent(s, ds.ws_free, 0));
    DET_HIP_CHECK(gemv_q16_any(w, x, y, m, k, nb, ds.ws, s));
    DET_HIP_CHECK(hipEventRecord(ds.ws_free, s));
    return 0;
}

int64_t det_gemv_i16_dev(const int16_t *w, const int16_t *x, int32_t *y, int64_t m, int64_t k, void *stream) {
    if (bad_dims(m, k, 1)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (m == 0) return 0;
    if (!y || ((!w || !x) && k > 0)) return set_err(DET_ERR_ARG, "null device pointer");
    hipStream_t s = (hipStream_t)stream;
    if (k == 0) DET_HIP_CHECK(zero_i32(y, (size_t)m, s));
    else DET_HIP_CHECK(det::launch_gemv_i16(w, x, y, (int)m, (int)k, s));
    return 0;
}
int64_t det_matmul_rmajor_f32_dev(const float *w, const float *x, float *y, int64_t rows, int64_t cols,
                                  void *stream) {
    if (rows < 0 || cols < 0 || rows >= (1LL << 31) || cols >= (1LL << 31))
        return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (rows == 0 || cols == 0) return 0;
    if (!w || !x || !y) return set_err(DET_ERR_ARG, "null device pointer");
    DET_HIP_CHECK(det::launch_rows_f32(w, x, y, rows, cols, det::F32_DOT, (hipStream_t)stream));
    return 0;
}
int64_t det_rows_metric_f32_dev(int64_t op, const float *w, const float *x, float *y, int64_t rows, int64_t cols,
                                void *stream) {
    if (op < DET_F32_DOT || op > DET_F32_LINF_V) return set_err(DET_ERR_ARG, "unknown f32 metric");
    if (rows < 0 || cols < 0 || rows >= (1LL << 31) || cols >= (1LL << 31))
        return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (rows == 0) return 0;
    if (!y) return set_err(DET_ERR_ARG, "null device pointer");
    hipStream_t s = (hipStream_t)stream;
    if (cols == 0) {   // every metric of two empty vectors is +0.0f
        DET_HIP_CHECK(zero_i32((int32_t *)y, (size_t)rows, s));
        return 0;
    }
    if (!w || !x) return set_err(DET_ERR_ARG, "null device pointer");
    DET_HIP_CHECK(det::launch_rows_f32(w, x, y, rows, cols, (int)op, s));
    return 0;
}
int64_t det_rows_metric_f32(int64_t op, const float *w, const float *x, float *y, int64_t rows, int64_t cols) {
    if (op < DET_F32_DOT || op > DET_F32_LINF_V) return set_err(DET_ERR_ARG, "unknown f32 metric");
    if (rows < 0 || cols < 0) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (rows == 0) return 0;
    if (!y) return set_err(DET_ERR_ARG, "null pointer");
    if (cols == 0) {
        memset(y, 0, (size_t)rows * 4);
        return 0;
    }
    if (!w || !x) return set_err(DET_ERR_ARG, "null pointer");
    return f32_rows_host(w, x, y, rows, cols, (int)op);
}
int64_t det_fft_q16(int64_t *re, int64_t *im, const int64_t *tw, int64_t logn, int64_t n, int64_t batch) {
    return fft_host((int64_t)(intptr_t)re, (int64_t)(intptr_t)im, (int64_t)(intptr_t)tw, logn, n, batch);
}
int64_t det_fft_q16_dev(int64_t *re, int64_t *im, const int64_t *tw, int64_t logn, int64_t n, int64_t batch,
                        void *stream) {
    const int64_t rc = fft_check(logn, n, batch);
    if (rc) return rc > 0 ? 0 : rc;
    if (!re || !im || (!tw && n >= 4)) return set_err(DET_ERR_ARG, "fft: null device pointer");
    return fft_dev_run(re, im, re, im, tw, (int)logn, batch, (hipStream_t)stream);
}
int64_t det_fft_q16_oop_dev(const int64_t *in_re, const int64_t *in_im, int64_t *out_re, int64_t *out_im,
                            const int64_t *tw, int64_t logn, int64_t n, int64_t batch, void *stream) {
    const int64_t rc = fft_check(logn, n, batch);
    if (rc) return rc > 0 ? 0 : rc;
    if (!in_re || !in_im || !out_re || !out_im || (!tw && n >= 4))
        return set_err(DET_ERR_ARG, "fft: null device pointer");
    const int64_t *ranges[4] = {in_re, in_im, out_re, out_im};
    const size_t bytes = (size_t)batch * n * 8;
    for (int a = 0; a < 2; ++a)
        for (int b = 2; b < 4; ++b) {
            const uintptr_t x = (uintptr_t)ranges[a], y = (uintptr_t)ranges[b];
            if (x != y && x < y + bytes && y < x + bytes)
                return set_err(DET_ERR_ARG, "fft: input and output overlap without being the same buffer");
        }
    return fft_dev_run(in_re, in_im, out_re, out_im, tw, (int)logn, batch, (hipStream_t)stream);
}
int64_t det_fft_workspace_bytes(int64_t logn, int64_t batch) {
    if (logn < 0 || logn > 30 || batch <= 0) return 0;
    return (int64_t)det::fft_workspace_bytes((int)logn, batch);
}
int64_t det_dot_dev(int64_t op, const void *a, const void *b, int64_t len, int32_t *out, void *stream) {
    if (op < det::DOT_Q16 || op > det::DOT_I16) return set_err(DET_ERR_ARG, "unknown dot op");
    if (len < 0 || len >= (1LL << 31)) return set_err(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (!out || ((!a || !b) && len > 0)) return set_err(DET_ERR_ARG, "null device pointer");
    DET_HIP_CHECK(det::launch_dot((int)op, a, b, len, (uint32_t *)out, (hipStream_t)stream));
    return 0;
}

// ---------------------------------------------------------------- runtime
// Teardown (the reference joins its thread pool at unload,
// runtime-support/mind_intrinsics.c:2066-2080).  Explicit, not an exit or
// unload hook: a handler that an atexit from this library registers runs at
// process exit as well as at dlclose, and HIP calls made during process exit
// abort under tools that intercept HIP (a profiler's per-thread state is
// gone by then).  Callers that unload the library call it before dlclose.
int64_t det_shutdown(void) {
    const int64_t rc = release_all();
    g_pool.stop();
    return rc;
}
const char *det_last_error(void) { return g_err; }
const char *det_version(void) { return "mind-det-mi355x 0.1 (gfx950)"; }

int64_t det_device_count(void) {
    int n = 0;
    DET_HIP_CHECK(hipGetDeviceCount(&n));
    return n;
}
int64_t det_set_device(int64_t d) {
    DET_HIP_CHECK(hipSetDevice((int)d));
    return 0;
}
// info: [0]=CU count [1]=max engine clock kHz [2]=global memory bytes
// [3]=LDS bytes per workgroup [4]=memory clock kHz [5]=memory bus width bits
int64_t det_device_info(int64_t *info, char *name, int64_t name_len) {
    int d = 0;
    DET_HIP_CHECK(hipGetDevice(&d));
    hipDeviceProp_t p;
    DET_HIP_CHECK(hipGetDeviceProperties(&p, d));
    if (info) {
        info[0] = p.multiProcessorCount;
        info[1] = p.clockRate;
        info[2] = (int64_t)p.totalGlobalMem;
        info[3] = (int64_t)p.sharedMemPerBlock;
        info[4] = p.memoryClockRate;
        info[5] = p.memoryBusWidth;
    }
    if (name && name_len > 0) {
        std::string s = p.name[0] ? std::string(p.name) + " " + p.gcnArchName : std::string(p.gcnArchName);
        size_t l = s.size() < (size_t)name_len - 1 ? s.size() : (size_t)name_len - 1;
        memcpy(name, s.data(), l);
        name[l] = 0;
    }
    return 0;
}
int64_t det_malloc(void **p, int64_t bytes) {
    if (!p || bytes < 0) return set_err(DET_ERR_ARG, "bad det_malloc arguments");
    *p = nullptr;
    if (bytes == 0) return 0;
    DET_HIP_CHECK(hipMalloc(p, (size_t)bytes));
    return 0;
}
int64_t det_free(void *p) {
    if (p) DET_HIP_CHECK(hipFree(p));
    return 0;
}
// The copies and the fill run on the null stream, which the library's
// non-blocking streams do not wait for: each returns only once its bytes
// have landed, so work queued afterwards on any stream sees them (hipMemcpy
// from pageable memory may return while the last DMA to the device is still
// in flight, and hipMemset is asynchronous for device memory).
int64_t det_memcpy_htod(void *dst, const void *src, int64_t bytes) {
    if (bytes > 0) {
        DET_HIP_CHECK(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice));
        DET_HIP_CHECK(hipStreamSynchronize(nullptr));
    }
    return 0;
}
int64_t det_memcpy_dtoh(void *dst, const void *src, int64_t bytes) {
    if (bytes > 0) DET_HIP_CHECK(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost));
    return 0;
}
int64_t det_memset_dev(void *dst, int64_t byte, int64_t bytes) {
    if (bytes > 0) {
        DET_HIP_CHECK(hipMemset(dst, (int)byte, (size_t)bytes));
        DET_HIP_CHECK(hipStreamSynchronize(nullptr));
    }
    return 0;
}
int64_t det_device_sync(void) {
    DET_HIP_CHECK(hipDeviceSynchronize());
    return 0;
}
int64_t det_stream_create(void **s) {
    DET_HIP_CHECK(hipStreamCreateWithFlags((hipStream_t *)s, hipStreamNonBlocking));
    return 0;
}
int64_t det_stream_destroy(void *s) {
    if (s) DET_HIP_CHECK(hipStreamDestroy((hipStream_t)s));
    return 0;
}
int64_t det_stream_sync(void *s) {
    DET_HIP_CHECK(hipStreamSynchronize((hipStream_t)s));
    return 0;
}
int64_t det_event_create(void **e) {
    DET_HIP_CHECK(hipEventCreate((hipEvent_t *)e));
    return 0;
}
int64_t det_event_destroy(void *e) {
    if (e) DET_HIP_CHECK(hipEventDestroy((hipEvent_t)e));
    return 0;
}
int64_t det_event_record(void *e, void *s) {
    DET_HIP_CHECK(hipEventRecord((hipEvent_t)e, (hipStream_t)s));
    return 0;
}
int64_t det_event_elapsed_ms(void *start, void *stop, float *ms) {
    DET_HIP_CHECK(hipEventSynchronize((hipEvent_t)stop));
    DET_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return 0;
}

}  // extern "C"
