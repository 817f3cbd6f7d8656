/*
 * det_driver.c -- a C caller of libmind_det_hip.so, shaped like the
 * reference's cross-node gate driver (tests/cross_substrate_identity/
 * xnode_driver.c:123-156): dlopen the library, dlsym the harness symbols
 * through i64-ABI function-pointer typedefs, regenerate the committed
 * workloads with the reference LCG, and print one SHA-256 per workload.
 *
 *   det_driver <libmind_det_hip.so> [libmind_det_gemmq_kn.so]
 *
 * Output lines: "<workload> <symbol> <sha256 hex>"; tests/test_c_driver.py
 * compares them with tests/golden/canaries.json.  Exit status: 0 when every
 * call returned 0, 1 on a failed call, 2 usage, 3 dlopen, 4 missing symbol.
 * It also includes include/mind_det.h and binds two entry points through
 * the header's own prototypes, so the header is checked as C.
 */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "mind_det.h"

/* ------------------------------------------------------------ SHA-256
 * FIPS 180-4, section 6.2 (written from the standard). */
typedef struct {
    uint32_t h[8];
    uint8_t buf[64];
    size_t fill;
    uint64_t bits;
} sha_t;

static const uint32_t SHA_K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static uint32_t rotr(uint32_t x, int r) { return (x >> r) | (x << (32 - r)); }

static void sha_block(sha_t *s, const uint8_t *p) {
    uint32_t w[64];
    for (int t = 0; t < 16; ++t)
        w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 | (uint32_t)p[4 * t + 2] << 8 | p[4 * t + 3];
    for (int t = 16; t < 64; ++t) {
        const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t v[8];
    memcpy(v, s->h, sizeof v);
    for (int t = 0; t < 64; ++t) {
        const uint32_t e = v[4], a = v[0];
        const uint32_t t1 = v[7] + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & v[5]) ^ (~e & v[6])) + SHA_K[t] + w[t];
        const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & v[1]) ^ (a & v[2]) ^ (v[1] & v[2]));
        memmove(v + 1, v, 7 * sizeof v[0]);
        v[4] += t1;
        v[0] = t1 + t2;
    }
    for (int i = 0; i < 8; ++i) s->h[i] += v[i];
}

static void sha_init(sha_t *s) {
    static const uint32_t h0[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(s->h, h0, sizeof h0);
    s->fill = 0;
    s->bits = 0;
}

static void sha_add(sha_t *s, const void *data, size_t n) {
    const uint8_t *p = (const uint8_t *)data;
    s->bits += (uint64_t)n * 8;
    while (n--) {
        s->buf[s->fill++] = *p++;
        if (s->fill == 64) {
            sha_block(s, s->buf);
            s->fill = 0;
        }
    }
}

static void sha_hex(sha_t *s, char out[65]) {
    const uint64_t bits = s->bits;
    const uint8_t one = 0x80, zero = 0;
    sha_add(s, &one, 1);
    while (s->fill != 56) sha_add(s, &zero, 1);
    uint8_t len[8];
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(bits >> (56 - 8 * i));
    sha_add(s, len, 8);
    for (int i = 0; i < 32; ++i) sprintf(out + 2 * i, "%02x", (s->h[i / 4] >> (24 - 8 * (i % 4))) & 0xff);
}

/* Hash of n int32 as little-endian bytes (the golden encoding). */
static void hash_i32(const int32_t *v, size_t n, char out[65]) {
    sha_t s;
    sha_init(&s);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t u = (uint32_t)v[i];
        const uint8_t b[4] = {(uint8_t)u, (uint8_t)(u >> 8), (uint8_t)(u >> 16), (uint8_t)(u >> 24)};
        sha_add(&s, b, 4);
    }
    sha_hex(&s, out);
}

static void hash_i64(int64_t r, char out[65]) {
    uint8_t b[8];
    for (int i = 0; i < 8; ++i) b[i] = (uint8_t)((uint64_t)r >> (8 * i));
    sha_t s;
    sha_init(&s);
    sha_add(&s, b, 8);
    sha_hex(&s, out);
}

/* ------------------------------------------------------------ inputs
 * The reference bench LCG: s <- s * 1664525 + 1013904223 (mod 2^64),
 * u32 = s >> 16; Q16 = (int32)u32 >> 12, int8 / int16 = top bits of u32. */
static uint64_t lcg;
static uint32_t draw(void) {
    lcg = lcg * 1664525u + 1013904223u;
    return (uint32_t)(lcg >> 16);
}
static int32_t draw_q16(void) { return (int32_t)draw() >> 12; }
static int8_t draw_i8(void) { return (int8_t)(draw() >> 16); }
static int16_t draw_i16(void) { return (int16_t)(draw() >> 16); }

#define SEED 0xDEADBEEFu
#define P(x) ((int64_t)(intptr_t)(x))

/* i64-ABI symbol shapes (xnode_driver.c:123-125) */
typedef int64_t (*fn3)(int64_t, int64_t, int64_t);
typedef int64_t (*fn5)(int64_t, int64_t, int64_t, int64_t, int64_t);
typedef int64_t (*fn6)(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t);

static void *lib;
static int failed;

static void *sym(void *h, const char *name) {
    void *f = dlsym(h, name);
    if (!f) {
        fprintf(stderr, "missing symbol %s\n", name);
        exit(4);
    }
    return f;
}

static void report(const char *id, const char *symbol, int64_t rc, const char *hex) {
    if (rc != 0) {
        const char *(*last)(void) = (const char *(*)(void))sym(lib, "det_last_error");
        fprintf(stderr, "%s via %s returned %lld: %s\n", id, symbol, (long long)rc, last());
        failed = 1;
    }
    printf("%s %s %s\n", id, symbol, hex);
}

/* --selftest: hash the driver's own Q16 64x64 A-then-B input and int32
 * 0..999, so the CPU tier can check the SHA-256 and the LCG without a GPU. */
static int selftest(void) {
    char hex[65];
    int32_t v[2 * 64 * 64];
    lcg = SEED;
    for (int i = 0; i < 2 * 64 * 64; ++i) v[i] = draw_q16();
    hash_i32(v, 2 * 64 * 64, hex);
    printf("lcg-q16-8192 %s\n", hex);
    for (int i = 0; i < 1000; ++i) v[i] = i - 500;
    hash_i32(v, 1000, hex);
    printf("ramp-1000 %s\n", hex);
    hash_i32(v, 0, hex);
    printf("empty %s\n", hex);
    return 0;
}

int main(int argc, char **argv) {
    if (argc == 2 && strcmp(argv[1], "--selftest") == 0) return selftest();
    if (argc < 2) {
        fprintf(stderr, "usage: %s <libmind_det_hip.so> [libmind_det_gemmq_kn.so]\n", argv[0]);
        return 2;
    }
    lib = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
        fprintf(stderr, "dlopen failed: %s\n", dlerror());
        return 3;
    }
    char hex[65];
    enum { G = 64, R = 256, L2 = 65536, LI16 = 4096 };

    /* gemm-i8-64x64x64 through gemmi8, gemmi8mt and the typed entry point */
    {
        int8_t *a = malloc(G * G), *b = malloc(G * G);
        int32_t *c = malloc(sizeof(int32_t) * G * G);
        lcg = SEED;
        for (int i = 0; i < G * G; ++i) a[i] = draw_i8();
        for (int i = 0; i < G * G; ++i) b[i] = draw_i8();
        static const char *names[] = {"gemmi8", "gemmi8mt", "__mind_blas_matmul_mm_i8_v"};
        for (int s = 0; s < 3; ++s) {
            memset(c, 0xA5, sizeof(int32_t) * G * G);
            const int64_t rc = ((fn6)sym(lib, names[s]))(P(a), P(b), P(c), G, G, G);
            hash_i32(c, G * G, hex);
            report("gemm-i8-64x64x64", names[s], rc, hex);
        }
        __typeof__(det_matmul_i8) *typed = (__typeof__(det_matmul_i8) *)sym(lib, "det_matmul_i8");
        memset(c, 0xA5, sizeof(int32_t) * G * G);
        const int64_t rc = typed(a, b, c, G, G, G);
        hash_i32(c, G * G, hex);
        report("gemm-i8-64x64x64", "det_matmul_i8", rc, hex);
        free(a), free(b), free(c);
    }
    /* gemm-q16-64x64x64: gemmq takes B^T [N][K]; gemmqmm and the bench
     * library's gemmq take B [K][N] */
    {
        int32_t *a = malloc(sizeof(int32_t) * G * G), *b = malloc(sizeof(int32_t) * G * G);
        int32_t *bt = malloc(sizeof(int32_t) * G * G), *c = malloc(sizeof(int32_t) * G * G);
        lcg = SEED;
        for (int i = 0; i < G * G; ++i) a[i] = draw_q16();
        for (int i = 0; i < G * G; ++i) b[i] = draw_q16();
        for (int k = 0; k < G; ++k)
            for (int j = 0; j < G; ++j) bt[j * G + k] = b[k * G + j];
        memset(c, 0xA5, sizeof(int32_t) * G * G);
        int64_t rc = ((fn6)sym(lib, "gemmq"))(P(a), P(bt), P(c), G, G, G);
        hash_i32(c, G * G, hex);
        report("gemm-q16-64x64x64", "gemmq", rc, hex);
        memset(c, 0xA5, sizeof(int32_t) * G * G);
        rc = ((fn6)sym(lib, "gemmqmm"))(P(a), P(b), P(c), G, G, G);
        hash_i32(c, G * G, hex);
        report("gemm-q16-fused-64x64x64", "gemmqmm", rc, hex);
        if (argc > 2) {
            void *kn = dlopen(argv[2], RTLD_NOW | RTLD_LOCAL);
            if (!kn) {
                fprintf(stderr, "dlopen failed: %s\n", dlerror());
                return 3;
            }
            memset(c, 0xA5, sizeof(int32_t) * G * G);
            rc = ((fn6)sym(kn, "gemmq"))(P(a), P(b), P(c), G, G, G);
            hash_i32(c, G * G, hex);
            report("gemm-q16-fused-64x64x64", "gemmq(kn)", rc, hex);
            dlclose(kn);
        }
        free(a), free(b), free(bt), free(c);
    }
    /* gemv-q16-256x256 through mmq and gemvq; gemv-i16-256x256 through mmi16 */
    {
        int32_t *w = malloc(sizeof(int32_t) * R * R), *x = malloc(sizeof(int32_t) * R);
        int32_t *y = malloc(sizeof(int32_t) * R);
        lcg = SEED;
        for (int i = 0; i < R * R; ++i) w[i] = draw_q16();
        for (int i = 0; i < R; ++i) x[i] = draw_q16();
        static const char *names[] = {"mmq", "gemvq"};
        for (int s = 0; s < 2; ++s) {
            memset(y, 0xA5, sizeof(int32_t) * R);
            const int64_t rc = ((fn5)sym(lib, names[s]))(P(w), P(x), P(y), R, R);
            hash_i32(y, R, hex);
            report("gemv-q16-256x256", names[s], rc, hex);
        }
        int16_t *w16 = malloc(sizeof(int16_t) * R * R), *x16 = malloc(sizeof(int16_t) * R);
        lcg = SEED;
        for (int i = 0; i < R * R; ++i) w16[i] = draw_i16();
        for (int i = 0; i < R; ++i) x16[i] = draw_i16();
        memset(y, 0xA5, sizeof(int32_t) * R);
        const int64_t rc = ((fn5)sym(lib, "mmi16"))(P(w16), P(x16), P(y), R, R);
        hash_i32(y, R, hex);
        report("gemv-i16-256x256", "mmi16", rc, hex);
        free(w), free(x), free(y), free(w16), free(x16);
    }
    /* scalar dots: the i64 result's 8 little-endian bytes are hashed */
    {
        int32_t *a = malloc(sizeof(int32_t) * L2), *b = malloc(sizeof(int32_t) * L2);
        lcg = SEED;
        for (int i = 0; i < L2; ++i) a[i] = draw_q16();
        for (int i = 0; i < L2; ++i) b[i] = draw_q16();
        hash_i64(((fn3)sym(lib, "dotq"))(P(a), P(b), L2), hex);
        report("dot-l2-q16", "dotq", 0, hex);
        hash_i64(((fn3)sym(lib, "dotl1q"))(P(a), P(b), L2), hex);
        report("dot-l1-q16", "dotl1q", 0, hex);
        int16_t *a16 = malloc(sizeof(int16_t) * LI16), *b16 = malloc(sizeof(int16_t) * LI16);
        lcg = SEED;
        for (int i = 0; i < LI16; ++i) a16[i] = draw_i16();
        for (int i = 0; i < LI16; ++i) b16[i] = draw_i16();
        hash_i64(((fn3)sym(lib, "doti16"))(P(a16), P(b16), LI16), hex);
        report("dot-i16-4096", "doti16", 0, hex);
        free(a), free(b), free(a16), free(b16);
    }
    __typeof__(det_shutdown) *shutdown = (__typeof__(det_shutdown) *)sym(lib, "det_shutdown");
    if (shutdown() != 0) failed = 1;
    dlclose(lib);
    return failed;
}
