/*
 * oracle/apus_oracle.h — TEST INFRASTRUCTURE ONLY: the CPU restatement of the
 * apus reference semantics for the FP8-block dequant -> BF16 GEMV/GEMM ->
 * routed-expert SwiGLU hot path. Used by tests/ as the parity checker and by
 * bench.py's cpu_baseline leg; never linked into or called by the product
 * library (apus-glm5.3-flash_amd/).
 *
 * Every function cites the reference file:line it restates. What each
 * function is checked against (the reference's known-answer tests and
 * golden vectors, closed forms, the reference's own C kernels built under
 * oracle/_ref) is exercised by the CPU test suite (tests/test_oracle_*.py).
 */
#ifndef APUS_ORACLE_H
#define APUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- codec (c/num.h) ------------------------------------------------------*/
float    apo_e4m3_f32(uint8_t c);          /* c/num.h:136-141 */
uint16_t apo_bf16_bits(float x);           /* c/num.h:153-159 */
float    apo_bf16_round(float x);          /* c/num.h:143-151 */
float    apo_bf16_f32(uint16_t b);         /* c/num.h:161-166 */
size_t   apo_nblocks(size_t n);            /* c/fp8blk.h:109-111 */

/* --- FP8 128x128-block dequant (c/fp8blk.h) ---------------------------------*/
/* scalar anchor, c/fp8blk.h:115-136 */
void apo_fp8blk_dequant(const uint8_t *w, const float *ws, uint16_t *out,
                        size_t O, size_t K);
/* threaded row partition, c/fp8blk.h:277-317 (bitwise == scalar) */
void apo_fp8blk_dequant_mt(const uint8_t *w, const float *ws, uint16_t *out,
                           size_t O, size_t K, int threads);

/* --- BF16 GEMV/GEMM, fp32 sequential-k (c/bf16.h) -----------------------------*/
/* scalar anchor, c/bf16.h:202-217 */
void apo_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                   size_t M, size_t O, size_t K);
/* timed CPU baseline: AVX2 staged products + 8 row chains / 4 shared m-rows,
 * contiguous pthread row partition (c/bf16.h:444-649, 739-767; c/pool.h:148-185).
 * Bitwise == apo_bf16_gemm at every thread count. Returns 0 (1 on OOM). */
int  apo_bf16_gemm_mt(const uint16_t *w, const uint16_t *x, uint16_t *y,
                      size_t M, size_t O, size_t K, int threads);
/* c/gdsa.h:525-534 CPU leg: dequant then GEMM (scalar or mt). */
int  apo_fp8blk_linear(const uint8_t *codes, const float *scales,
                       const uint16_t *x, uint16_t *y,
                       size_t M, size_t O, size_t K, int threads);
/* Test helper for the tolerance floor: A[m,o] = sum_k |W[o,k] * x[m,k]| in
 * f64 over the bf16 weights (not a reference function). */
void apo_bf16_gemm_absdot(const uint16_t *w, const uint16_t *x, double *a,
                          size_t M, size_t O, size_t K);

/* --- routed expert SwiGLU + combine (c/gmoe.h, c/gmhc.h) ---------------------*/
float apo_sigmoid_np(float x);             /* c/gmhc.h:157-160 */
float apo_pw_sum(const float *a, size_t n);/* c/gmhc.h:165-185 */
/* c/gmoe.h:175-189: k passes of strict-greater argmax, ties -> lower index */
void  apo_topk_stable(const float *row, int n, int k, int32_t *idx);
/* c/gmoe.h:168-173: one gate-row fp32 dot, ascending k, mul then add */
float apo_gate_dot(const uint16_t *wrow, const uint16_t *x, size_t k);
/* c/gmoe.h:191-208: the reference router (sigmoid scores, selection-only
 * bias, stable top-k, pairwise-sum normalization x route_scale) */
void  apo_gmoe_router(const uint16_t *gate_w, const float *gate_bias, int E,
                      size_t dim, int topk, float route_scale, const uint16_t *x,
                      float *scores, int32_t *idx, float *w);
/* the same from given logits (everything after the gate dots) */
void  apo_gmoe_router_from_logits(const float *logits, const float *gate_bias, int E,
                                  int topk, float route_scale, float *scores,
                                  int32_t *idx, float *w);
/* c/gmoe.h:210-227 on BF16 payloads: g,u GEMVs, clamps, two bf16 rounds,
 * down GEMV. g_out/u_out/h_out optional (NULL to skip). */
int   apo_swiglu_expert(const uint16_t *wg, const uint16_t *wu,
                        const uint16_t *wd, const uint16_t *x,
                        size_t dim, size_t inter, float limit,
                        uint16_t *out, uint16_t *g_out, uint16_t *u_out,
                        uint16_t *h_out, int threads);

/* Expert slab layout (c/gcache.h:852-861): gate.w | gate.s | up.w | up.s |
 * down.w | down.s. Byte offsets of the six members and the slab size. */
typedef struct {
    size_t gw, gs, uw, us, dw, ds, bytes;
} ApoSlabLayout;
ApoSlabLayout apo_slab_layout(size_t dim, size_t inter);

/* Dequant-on-fill of one slab into a BF16 payload [gate | up | down]
 * (c/gcache.h:413-426). payload: 3*inter*dim u16. */
void apo_slab_dequant(const uint8_t *slab, size_t dim, size_t inter,
                      uint16_t *payload, int threads);

/* Routed MoE for T tokens over a slab bank, the reference combine
 * (c/gmoe.h:294-320 without router/shared expert): per token, experts in
 * ASCENDING id, contrib = bf16(out_e * w), y = bf16(y + contrib).
 * slabs[e] = host pointer to expert e's slab; idx/w [T, topk]. Each used
 * expert is dequantized once (payload cache over the call). out [T, dim].
 * expert_out (optional) [T, topk, dim]: out_e per (token, slot). */
int apo_moe_forward(const uint8_t *const *slabs, int n_experts,
                    size_t dim, size_t inter, float limit,
                    const uint16_t *x, size_t T, const int32_t *idx,
                    const float *w, int topk, uint16_t *out,
                    uint16_t *expert_out, int threads);

/* apo_moe_forward plus the shared expert (c/gmoe.h:325-336): after the
 * routed combine, out = bf16(y + sh) with sh the shared expert's bf16
 * output on the shared slab (same layout; intermediate = inter, as
 * n_shared_experts = 1 gives, c/gmodel.h:963-964). shared_out (optional)
 * [T, dim]: sh. */
int apo_moe_forward_shared(const uint8_t *const *slabs, int n_experts,
                           const uint8_t *shared_slab, size_t dim, size_t inter,
                           float limit, const uint16_t *x, size_t T, const int32_t *idx,
                           const float *w, int topk, uint16_t *out,
                           uint16_t *expert_out, uint16_t *shared_out, int threads);

/* The same result computed expert by expert (each used expert dequantized
 * once, its tokens as one M-row GEMM per matrix; bitwise equal to
 * apo_moe_forward, or to apo_moe_forward_shared with shared_slab non-NULL,
 * by the M-independence of c/bf16.h:27-37), for checks at full size.
 * expert_out (optional) [T, topk, dim]: out_e per kept (token, slot); the
 * entries of dropped slots are left as they are. */
int apo_moe_forward_grouped(const uint8_t *const *slabs, int n_experts,
                            const uint8_t *shared_slab, size_t dim, size_t inter,
                            float limit,
                            const uint16_t *x, size_t T, const int32_t *idx,
                            const float *w, int topk, uint16_t *out,
                            uint16_t *expert_out, int threads);

/* Test yardstick, not a reference function: apo_moe_forward_grouped with
 * every GEMM dot product summed in f64 (then rounded to f32 and bf16 at
 * the reference's rounding points; SwiGLU and combine unchanged), free of
 * any fp32 summation order. */
int apo_moe_chain64_grouped(const uint8_t *const *slabs, int n_experts,
                            const uint8_t *shared_slab, size_t dim, size_t inter,
                            float limit,
                            const uint16_t *x, size_t T, const int32_t *idx,
                            const float *w, int topk, uint16_t *out,
                            uint16_t *expert_out, int threads);

/* Test helper for the combine's tolerance floor (not a reference
 * function): out as apo_moe_forward_grouped, and floor_out [T, dim] f64 =
 * sum over the token's kept pairs of |w_e| * sum_i |h_i * wd_e[j,i]|, the
 * expert-output floor (the down GEMM's term magnitudes, h the reference's)
 * carried through the combine weights. */
int apo_moe_floor_grouped(const uint8_t *const *slabs, int n_experts,
                          const uint8_t *shared_slab, size_t dim, size_t inter,
                          float limit,
                          const uint16_t *x, size_t T, const int32_t *idx,
                          const float *w, int topk, uint16_t *out,
                          double *floor_out, int threads);

/* Harness routing (configs 2-4 of the bench spec; NOT the reference's
 * sigmoid router): idx = stable top-k of logits (ties -> lower index),
 * w = softmax over the k selected logits: m = logit[idx[0]],
 * e_j = expf(l_j - m), s = sum_j e_j (ascending j), w_j = e_j / s. */
void apo_route_softmax(const float *logits, int E, int k, int32_t *idx,
                       float *w);

/* Row-partitioned thread count actually used for nthreads <= 0 (= online
 * CPUs, clamped to 64). */
int apo_default_threads(void);

#ifdef __cplusplus
}
#endif
#endif /* APUS_ORACLE_H */
