/*
 * test_boundary.c — a compiled C caller of the backend boundary, linked the
 * way the engine links it: engine_tu.c (the engine's own hook table; built
 * with APUS_GHIP_LINKED, so no stubs) + libapus_ghip.so, checked against
 * the CPU restatement in oracle/ (liboracle.so). The analog of the
 * reference's GPU gate tests/m7b/test_gkernels.c:77-324 for this backend.
 *
 *   - the library writes the ENGINE's table (its weak definition is
 *     interposed by the engine's strong one): disable clears dummy entries
 *     the program put there, enable fills them;
 *   - without a usable device (the CPU box) enable declines with a reason
 *     and the table stays all-NULL (every call site runs its CPU kernel);
 *   - with the device: the floors and the M gate decline without touching
 *     y (APUS_GHIP_FP8_MIN_KB = 16384 keeps config 0's 8 MiB weight on the
 *     CPU, APUS_GHIP_MAX_M = 4 keeps M = 5), the hooks produce configs 0
 *     (direct entry) and 1 (M = 1, 2, 4) and a BF16 GEMM within the
 *     contract tolerance of the oracle, and disable clears the table.
 *
 * Usage: test_boundary [--expect-gpu]. Exit 0 = every check passed.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "apus_oracle.h"
#include "apus_synth.h"
#include "backend_hip.h"

static int g_fail;

#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            printf("FAIL %s:%d: ", __FILE__, __LINE__);    \
            printf(__VA_ARGS__);                           \
            printf("\n");                                  \
            g_fail = 1;                                    \
        }                                                  \
    } while (0)

static int dummy_bf16(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M,
                      size_t O, size_t K) {
    (void)w; (void)x; (void)y; (void)M; (void)O; (void)K;
    return 1;
}

static int dummy_fp8(const uint8_t *c, const float *s, const uint16_t *x, uint16_t *y,
                     size_t M, size_t O, size_t K) {
    (void)c; (void)s; (void)x; (void)y; (void)M; (void)O; (void)K;
    return 1;
}

static long bf16_ord(uint16_t b) {
    long m = b & 0x7fff;
    return (b & 0x8000) ? -m : m;
}

/* the contract tolerance (tests/tolerance.py): <= 1 bf16 ulp on >= 99.9%
 * of elements, |got - ref| / max(|ref|, floor) <= 1e-2 */
static void tolerance(const char *what, const uint16_t *got, const uint16_t *ref,
                      const double *floor, size_t n) {
    size_t le1 = 0;
    double maxrel = 0.0;
    for (size_t i = 0; i < n; i++) {
        long d = labs(bf16_ord(got[i]) - bf16_ord(ref[i]));
        le1 += d <= 1;
        double g = apo_bf16_f32(got[i]), r = apo_bf16_f32(ref[i]);
        double den = fmax(fabs(r), floor[i]);
        double rel = den > 0 ? fabs(g - r) / den : (g == r ? 0.0 : INFINITY);
        if (!(rel <= maxrel)) maxrel = rel;
    }
    double frac = n ? (double)le1 / (double)n : 1.0;
    printf("  %-34s n=%zu le1ulp=%.6f max_rel=%.2e\n", what, n, frac, maxrel);
    CHECK(frac >= 0.999 && maxrel <= 1e-2, "%s outside the tolerance", what);
}

typedef struct {
    size_t O, K, M;
    uint8_t *codes;
    float *scales;
    uint16_t *w;            /* dequantized weights (oracle) */
    uint16_t *x, *ref;
    double *floor;
} Case;

/* config inputs from the shared generator (include/apus_synth.h), the
 * oracle's output and the 2^-8 sum|w x| floor */
static Case make_case(size_t O, size_t K, size_t M, uint64_t seed) {
    Case c = {O, K, M, NULL, NULL, NULL, NULL, NULL, NULL};
    size_t nsb = apo_nblocks(O) * apo_nblocks(K);
    c.codes = malloc(O * K);
    c.scales = malloc(nsb * sizeof(float));
    c.w = malloc(O * K * 2);
    c.x = malloc(M * K * 2);
    c.ref = malloc(M * O * 2);
    c.floor = malloc(M * O * sizeof(double));
    if (!c.codes || !c.scales || !c.w || !c.x || !c.ref || !c.floor || M > 5) {
        printf("FAIL: out of memory\n");
        exit(1);
    }
    apus_synth_fp8_codes(c.codes, O * K, seed, 10, 0);
    apus_synth_scales(c.scales, nsb, seed, 11, 1e-4f, 1e-2f);
    apus_synth_bf16_normal(c.x, M * K, seed, 12, 0);
    apo_fp8blk_dequant_mt(c.codes, c.scales, c.w, O, K, 0);
    apo_bf16_gemm_mt(c.w, c.x, c.ref, M, O, K, 0);
    apo_bf16_gemm_absdot(c.w, c.x, c.floor, M, O, K);
    for (size_t i = 0; i < M * O; i++) c.floor[i] *= 1.0 / 256.0;
    return c;
}

static void free_case(Case *c) {
    free(c->codes); free(c->scales); free(c->w); free(c->x); free(c->ref); free(c->floor);
}

/* y prefilled with a sentinel: a declined call must leave it untouched */
static int untouched(const uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (y[i] != 0x7E57) return 0;
    return 1;
}

int main(int argc, char **argv) {
    int expect_gpu = argc > 1 && strcmp(argv[1], "--expect-gpu") == 0;
    char err[256] = "";
    setvbuf(stdout, NULL, _IONBF, 0);             /* every line out, even on an abort */

    /* the table is the engine's; the library writes it through the
     * interposed symbol (disable clears what the program put there) */
    CHECK(!apus_ghip_hooks.bf16_gemm && !apus_ghip_hooks.fp8blk_linear,
          "hook table not all-NULL at start");
    apus_ghip_hooks.bf16_gemm = dummy_bf16;
    apus_ghip_hooks.fp8blk_linear = dummy_fp8;
    apus_ghip_disable();
    CHECK(!apus_ghip_hooks.bf16_gemm && !apus_ghip_hooks.fp8blk_linear,
          "apus_ghip_disable did not clear the engine's table: the library "
          "writes another copy");

    setenv("APUS_GHIP_FP8_MIN_KB", "16384", 1);
    setenv("APUS_GHIP_MAX_M", "4", 1);
    int rc = apus_ghip_enable(err, sizeof err);
    if (rc != 0) {
        printf("enable declined: rc=%d (%s)\n", rc, err);
        CHECK(!expect_gpu, "a device was expected");
        CHECK(err[0] != 0, "no reason given");
        CHECK(apus_ghip_is_enabled() == 0, "is_enabled after a declined enable");
        CHECK(!apus_ghip_hooks.bf16_gemm && !apus_ghip_hooks.fp8blk_linear,
              "hooks set after a declined enable");
        printf(g_fail ? "FAIL\n" : "PASS (no device: the CPU kernels run)\n");
        return g_fail;
    }
    CHECK(apus_ghip_is_enabled() == 1, "not enabled");
    CHECK(apus_ghip_hooks.bf16_gemm && apus_ghip_hooks.fp8blk_linear,
          "enable did not fill the engine's table");
    if (g_fail) {
        printf("FAIL\n");
        return 1;
    }

    /* config 0 (W [2048, 4096], 8 MiB of codes): below the 16 MiB floor the
     * hook declines; the direct entry point has no floors */
    Case c0 = make_case(2048, 4096, 1, 0xC0);
    uint16_t *y = malloc(5 * 16384 * 2);          /* the largest case: M = 5 */
    for (size_t i = 0; i < 2048; i++) y[i] = 0x7E57;
    rc = apus_ghip_hooks.fp8blk_linear(c0.codes, c0.scales, c0.x, y, 1, 2048, 4096);
    CHECK(rc != 0 && untouched(y, 2048), "config 0 under the floor: rc=%d", rc);
    rc = apus_ghip_fp8blk_linear(c0.codes, c0.scales, c0.x, y, 1, 2048, 4096);
    CHECK(rc == 0, "direct config 0: %s", apus_ghip_last_error());
    if (rc == 0) tolerance("config 0 M=1 (direct entry)", y, c0.ref, c0.floor, 2048);

    /* BF16 hook on the dequantized config-0 weights, M = 3 */
    {
        uint16_t x3[3 * 4096], r3[3 * 2048];
        double f3[3 * 2048];
        apus_synth_bf16_normal(x3, 3 * 4096, 0xB3, 12, 0);
        apo_bf16_gemm_mt(c0.w, x3, r3, 3, 2048, 4096, 0);
        apo_bf16_gemm_absdot(c0.w, x3, f3, 3, 2048, 4096);
        for (size_t i = 0; i < 3 * 2048; i++) f3[i] *= 1.0 / 256.0;
        rc = apus_ghip_hooks.bf16_gemm(c0.w, x3, y, 3, 2048, 4096);
        CHECK(rc == 0, "bf16 hook: %s", apus_ghip_last_error());
        if (rc == 0) tolerance("bf16 hook [2048, 4096] M=3", y, r3, f3, 3 * 2048);
    }
    free_case(&c0);

    /* config 1 (W [16384, 4096], 64 MiB) through the hook, M = 1, 2, 4;
     * M = 5 is above APUS_GHIP_MAX_M and declines */
    for (size_t M = 1; M <= 5; M = M == 2 ? 4 : M + 1) {
        Case c1 = make_case(16384, 4096, M, 0xC1);
        for (size_t i = 0; i < M * 16384; i++) y[i] = 0x7E57;
        rc = apus_ghip_hooks.fp8blk_linear(c1.codes, c1.scales, c1.x, y, M, 16384, 4096);
        if (M == 5) {
            CHECK(rc != 0 && untouched(y, M * 16384), "M=5 above the M gate: rc=%d", rc);
        } else {
            char what[64];
            snprintf(what, sizeof what, "config 1 M=%zu (hook)", M);
            CHECK(rc == 0, "%s: %s", what, apus_ghip_last_error());
            if (rc == 0) tolerance(what, y, c1.ref, c1.floor, M * 16384);
        }
        free_case(&c1);
    }
    CHECK(apus_ghip_offload_fp8blk() >= 3 && apus_ghip_offload_bf16() >= 1,
          "offload counters fp8 %llu bf16 %llu",
          (unsigned long long)apus_ghip_offload_fp8blk(),
          (unsigned long long)apus_ghip_offload_bf16());
    free(y);

    apus_ghip_disable();
    CHECK(!apus_ghip_hooks.bf16_gemm && !apus_ghip_hooks.fp8blk_linear &&
          apus_ghip_is_enabled() == 0, "disable left the table set");
    printf(g_fail ? "FAIL\n" : "PASS\n");
    return g_fail;
}
