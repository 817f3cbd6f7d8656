/*
 * libmind_det_gemmq_kn.so -- the `gemmq` symbol with B un-transposed.
 *
 * The reference binds the name `gemmq` to two different layouts, depending
 * on which MIND source was compiled into the .so it dlopens:
 *   - the golden gate's wrapper takes B TRANSPOSED, bt[N][K]
 *     (tests/cross_substrate_identity.rs:82-94); libmind_det_hip.so exports
 *     that form;
 *   - the Q16 GEMM benches wrap the fused intrinsic and pass B as K x N
 *     row-major (benches/det_matmul_q16.rs:111-122, :278;
 *     benches/det_matmul_q16_mt.rs:90-98, :239).
 * One library cannot export both under one name, so the bench form lives
 * here: dlopen this file instead of libmind_det_hip.so for those two benches.
 * It links libmind_det_hip.so (found next to it through $ORIGIN) and
 * forwards to its __mind_blas_matmul_mm_q16_v.
 */
#include <stdint.h>

int64_t __mind_blas_matmul_mm_q16_v(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n);

int64_t gemmq(int64_t a, int64_t b, int64_t c, int64_t m, int64_t k, int64_t n) {
    return __mind_blas_matmul_mm_q16_v(a, b, c, m, k, n);
}
