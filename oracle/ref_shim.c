/*
 * oracle/ref_shim.c — TEST INFRASTRUCTURE ONLY. Instantiates the reference
 * engine's own CPU kernels (header-only C under /root/reference/c, built by
 * oracle/Makefile into oracle/_ref/libapusref.so) and exports them under
 * stable names so the tests can check the C restatement (oracle/apus_oracle.c)
 * against the real reference, and bench.py can time the reference CPU path
 * ("cpu_baseline.kind": "reference").
 *
 * Nothing here is product code and no reference source is copied: this file
 * only #includes the reference headers where they lie and forwards calls.
 *
 * Instantiated reference symbols (file:line in the reference tree):
 *   apus_e4m3_dequant_f32        c/num.h:136-141
 *   apus_bf16_bits / _round      c/num.h:143-159
 *   apus_fp8blk_dequant_scalar   c/fp8blk.h:115-136
 *   apus_fp8blk_dequant_mt       c/fp8blk.h:277-317
 *   apus_bf16_gemm_scalar        c/bf16.h:213-217
 *   apus_bf16_gemm_mt            c/bf16.h:739-767 (AVX2 rows 578-634 + pool)
 *   apus_gmhc_sigmoid            c/gmhc.h:157-160
 *   apus_gmhc_pw_sum             c/gmhc.h:165-185
 *   apus_gmoe_topk_stable        c/gmoe.h:175-189
 *   apus_gmoe_expert             c/gmoe.h:210-227
 *   apus_gmoe_router             c/gmoe.h:191-208
 *   apus_gmoe_forward2           c/gmoe.h:265-337 (router, routed experts,
 *                                shared expert; with its scratch init/free)
 */
#define APUS_GMHC_IMPLEMENTATION
#define APUS_GMOE_IMPLEMENTATION
#define APUS_BF16_IMPLEMENTATION
#define APUS_FP8BLK_IMPLEMENTATION
#include "gmhc.h"
#include "gmoe.h"
#include "bf16.h"
#include "fp8blk.h"

#include <stdlib.h>
#include <string.h>

#define REF_API __attribute__((visibility("default")))

REF_API float ref_e4m3_f32(uint8_t c) { return apus_e4m3_dequant_f32(c); }
REF_API uint16_t ref_bf16_bits(float x) { return apus_bf16_bits(x); }
REF_API float ref_bf16_round(float x) { return apus_bf16_round(x); }
REF_API float ref_sigmoid(float x) { return apus_gmhc_sigmoid(x); }
REF_API float ref_pw_sum(const float *a, size_t n) {
    return apus_gmhc_pw_sum(a, n);
}
REF_API void ref_topk_stable(const float *row, int n, int k, int32_t *idx) {
    apus_gmoe_topk_stable(row, n, k, idx);
}

REF_API void ref_fp8blk_dequant_scalar(const uint8_t *w, const float *ws,
                                       uint16_t *out, size_t O, size_t K) {
    apus_fp8blk_dequant_scalar(w, ws, out, O, K);
}
REF_API void ref_fp8blk_dequant_mt(const uint8_t *w, const float *ws,
                                   uint16_t *out, size_t O, size_t K) {
    apus_fp8blk_dequant_mt(w, ws, out, O, K);
}
REF_API void ref_bf16_gemm_scalar(const uint16_t *w, const uint16_t *x,
                                  uint16_t *y, size_t M, size_t O, size_t K) {
    apus_bf16_gemm_scalar(w, x, y, M, O, K);
}
/* xf scratch is allocated here (M*K floats), as every reference caller does
 * with its own scratch. */
REF_API int ref_bf16_gemm_mt(const uint16_t *w, const uint16_t *x,
                             uint16_t *y, size_t M, size_t O, size_t K) {
    float *xf = (float *)malloc((M * K > 0 ? M * K : 1) * sizeof(float));
    if (!xf) return 1;
    apus_bf16_gemm_mt(w, x, xf, y, M, O, K);
    free(xf);
    return 0;
}
/* c/gdsa.h:525-534 CPU leg: dequant_mt into wbuf, then gemm_mt. */
REF_API int ref_fp8blk_linear_mt(const uint8_t *codes, const float *scales,
                                 const uint16_t *x, uint16_t *y,
                                 size_t M, size_t O, size_t K) {
    uint16_t *wbuf = (uint16_t *)malloc((O * K > 0 ? O * K : 1) * 2);
    float *xf = (float *)malloc((M * K > 0 ? M * K : 1) * sizeof(float));
    if (!wbuf || !xf) { free(wbuf); free(xf); return 1; }
    apus_fp8blk_dequant_mt(codes, scales, wbuf, O, K);
    apus_bf16_gemm_mt(wbuf, x, xf, y, M, O, K);
    free(wbuf);
    free(xf);
    return 0;
}
/* One routed expert on BF16 payloads (c/gmoe.h:210-227). */
REF_API int ref_gmoe_expert(const uint16_t *wg, const uint16_t *wu,
                            const uint16_t *wd, const uint16_t *x,
                            size_t dim, size_t inter, float limit,
                            uint16_t *out) {
    size_t mk = dim > inter ? dim : inter;
    uint16_t *g = (uint16_t *)malloc(inter * 2);
    uint16_t *u = (uint16_t *)malloc(inter * 2);
    uint16_t *h = (uint16_t *)malloc(inter * 2);
    float *xf = (float *)malloc(mk * sizeof(float));
    if (!g || !u || !h || !xf) {
        free(g); free(u); free(h); free(xf);
        return 1;
    }
    apus_gmoe_expert(wg, wu, wd, x, dim, inter, limit, out, g, u, h, xf);
    free(g); free(u); free(h); free(xf);
    return 0;
}
REF_API int ref_pool_threads(void) { return apus_pool_threads(); }
/* The per-token router (c/gmoe.h:191-208); scores [E] out. */
REF_API void ref_gmoe_router(const uint16_t *gate_w, const float *gate_bias, int E,
                             size_t dim, int topk, float route_scale,
                             const uint16_t *x, float *scores, int32_t *idx, float *w) {
    ApusGmoeRouterW r;
    r.E = E;
    r.topk = topk;
    r.dim = dim;
    r.route_scale = route_scale;
    r.gate_w = gate_w;
    r.gate_bias = gate_bias;
    float *b = (float *)malloc((size_t)(E > 0 ? E : 1) * sizeof(float));
    apus_gmoe_router(&r, x, scores, idx, w, b);
    free(b);
}
/* The whole MoE sublayer (c/gmoe.h:265-337) on BF16 payloads: per token
 * the router, the routed experts in ascending id, then the shared expert
 * added last. payloads[e] = expert e's [gate | up | down] (inter rows each);
 * shared = the shared expert's payload (sinter rows). x / out [s, dim];
 * idx_out / w_out [s, topk] (the router's picks; may be NULL). */
REF_API void ref_gmoe_forward2(const uint16_t *const *payloads, int E, size_t dim,
                               size_t inter, const uint16_t *shared, size_t sinter,
                               float limit, const uint16_t *gate_w,
                               const float *gate_bias, int topk, float route_scale,
                               const uint16_t *x, size_t s, uint16_t *out,
                               int32_t *idx_out, float *w_out) {
    const uint16_t **eg = (const uint16_t **)malloc((size_t)E * sizeof(*eg));
    const uint16_t **eu = (const uint16_t **)malloc((size_t)E * sizeof(*eu));
    const uint16_t **ed = (const uint16_t **)malloc((size_t)E * sizeof(*ed));
    for (int e = 0; e < E; e++) {
        eg[e] = payloads[e];
        eu[e] = payloads[e] + inter * dim;
        ed[e] = payloads[e] + 2 * inter * dim;
    }
    ApusGmoeW w;
    memset(&w, 0, sizeof w);
    w.router.E = E;
    w.router.topk = topk;
    w.router.dim = dim;
    w.router.route_scale = route_scale;
    w.router.gate_w = gate_w;
    w.router.gate_bias = gate_bias;
    w.inter = inter;
    w.eg = eg;
    w.eu = eu;
    w.ed = ed;
    w.sg = shared;
    w.su = shared + sinter * dim;
    w.sd = shared + 2 * sinter * dim;
    w.sinter = sinter;
    w.limit = limit;
    ApusGmoeInterm im;
    memset(&im, 0, sizeof im);
    im.router_idx = idx_out;
    im.router_w = w_out;
    ApusGmoeScratch sc;
    apus_gmoe_scratch_init(&sc, &w, s);
    apus_gmoe_forward2(&w, x, s, out, &im, &sc, NULL);
    apus_gmoe_scratch_free(&sc);
    free(eg); free(eu); free(ed);
}
