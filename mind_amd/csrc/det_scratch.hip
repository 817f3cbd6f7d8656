// det_scratch.hip -- det_matmul_scratch_dev: the workspace GEMM entry point
// for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// It is det_matmul_ws_dev with the workspace taken from `scratch`, a fixed
// array of DET_SCRATCH_BYTES compiled into the library: every GPU the
// library runs on holds its own copy for the life of the process.  The
// limb GEMMs' preps write every workspace byte they read, so the scratch
// needs no clearing between calls.  All calls on one GPU share that GPU's
// array: calls that overlap on one GPU (two streams, or two host threads)
// race and must be ordered by the caller.
#include <mutex>

#include "det_common.h"
#include "det_kernels.h"
#include "../../include/mind_det.h"

static __device__ __align__(256) unsigned char scratch[DET_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEV = 64;

// Device address of `scratch` on each device.  In host code the array's name
// is only a handle for the symbol lookup, never a device address.
void *g_scratch_ptr[MAX_DEV];
std::mutex g_scratch_mu;

// Looks the array up once per device, with that device current.
int64_t scratch_on_current_device(void **out) {
    int d = 0;
    hipError_t e = hipGetDevice(&d);
    if (e != hipSuccess) return det_fail_hip(e, "hipGetDevice");
    if (d < 0 || d >= MAX_DEV) return det_fail(DET_ERR_DEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[d]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return det_fail_hip(e, "hipGetSymbolAddress(scratch)");
        if (!p) return det_fail(DET_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[d] = p;
    }
    *out = g_scratch_ptr[d];
    return 0;
}

__global__ void scratch_zero_i32(int32_t *p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

extern "C" int64_t det_matmul_scratch_dev(int64_t op, const void *a, const void *b, int32_t *c, int64_t m, int64_t k,
                                          int64_t n, void *stream) {
    constexpr int64_t DIM_MAX = 0x7fffffff;
    if (m < 0 || k < 0 || n < 0 || m > DIM_MAX || k > DIM_MAX || n > DIM_MAX)
        return det_fail(DET_ERR_ARG, "dimension out of range [0, 2^31)");
    if (op != DET_OP_I8 && op != DET_OP_I16 && op != DET_OP_Q16) return det_fail(DET_ERR_ARG, "unknown op");
    if (m == 0 || n == 0) return 0;
    if (!a || !b || !c) return det_fail(DET_ERR_ARG, "null device pointer");
    const int M = (int)m, N = (int)n, K = (int)k;
    hipStream_t s = (hipStream_t)stream;
    if (K == 0) {
        // the exact sum over no terms
        const size_t cnt = (size_t)m * (size_t)n;
        hipLaunchKernelGGL(scratch_zero_i32, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s, c, cnt);
        DET_HIP_CHECK(hipGetLastError());
        return 0;
    }
    if (op == DET_OP_I8) {
        // int8 uses the scratch only to repack operands into padded panels
        // (off the 16-byte grid, or small grids the edge kernel would
        // underfill); beyond the scratch it takes the byte-load or edge
        // kernel, which need no workspace
        const bool aligned = (((uintptr_t)a | (uintptr_t)b) & 15) == 0;
        const size_t need8 = det::i8_workspace_bytes(M, N, K, aligned);
        void *ws8 = nullptr;
        if (need8 && need8 <= (size_t)DET_SCRATCH_BYTES) {
            const int64_t rc = scratch_on_current_device(&ws8);
            if (rc) return rc;
        }
        DET_HIP_CHECK(det::launch_gemm_i8((const int8_t *)a, (const int8_t *)b, c, M, N, K, ws8, s));
        return 0;
    }
    const size_t need = op == DET_OP_I16 ? det::i16_workspace_bytes(M, N, K) : det::q16_workspace_bytes(M, N, K);
    if (need > (size_t)DET_SCRATCH_BYTES)
        return det_fail(DET_ERR_ARG, "shape needs more workspace than the fixed scratch (DET_SCRATCH_BYTES); "
                                     "use det_matmul_ws_dev");
    void *ws = nullptr;
    const int64_t rc = scratch_on_current_device(&ws);
    if (rc) return rc;
    if (op == DET_OP_I16) DET_HIP_CHECK(det::launch_gemm_i16((const int16_t *)a, (const int16_t *)b, c, M, N, K, ws, s));
    else DET_HIP_CHECK(det::launch_gemm_q16((const int32_t *)a, (const int32_t *)b, c, M, N, K, false, ws, s));
    return 0;
}
