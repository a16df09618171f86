/*
 * include/backend_hip.h — MI355X (gfx950) backend for the apus GLM-5.3-Flash
 * dense FP8-block / BF16 compute and the routed-expert SwiGLU. Pure C ABI,
 * implemented by libapus_ghip.so (C host layer + hand-written HIP kernels).
 *
 * DROP-IN BOUNDARY. The first block mirrors the reference's Metal backend
 * interface c/backend_gmetal.h one for one (the g-prefix "gmetal" becomes
 * "ghip"); the engine's call sites (c/bf16.h:717-719, 743-745 and
 * c/gdsa.h:529-531) try the hook first and fall back to the pinned CPU
 * kernel when the pointer is NULL or the call returns nonzero — per-op
 * fail-soft, never a crash. The hook table is all-NULL until
 * apus_ghip_enable() succeeds.
 *
 * NUMERICS CONTRACT (differs from the Metal backend's, which is bitwise):
 *   - FP8-block dequant (apus_ghip_fp8blk_dequant*, and every kernel that
 *     consumes FP8 weights): BITWISE equal to c/fp8blk.h
 *     (bf16_rne(e4m3(code) * scale), one fp32 multiply; NaN codes 0x7F/0xFF
 *     decode as +-480 like c/num.h:136-141).
 *   - GEMV/GEMM outputs: the products of bf16 operands are exact in fp32 and
 *     are accumulated in fp32 in a blocked order (MFMA k-slices and a fixed
 *     cross-wave reduction) instead of the reference's strictly sequential k
 *     (c/bf16.h:27-37). Results agree with the CPU kernels to <= 1 bf16 ulp
 *     on >= 99.9% of elements, max relative error 1e-2 against
 *     max(|ref|, 2^-8 * sum_k |w*x|). Deterministic run to run.
 *   - SwiGLU / combine: the reference's clamp order, bf16 roundings and
 *     ascending-expert bf16-per-add combine (c/gmoe.h:210-227, 307-320),
 *     the shared expert added last (c/gmoe.h:325-336). The SwiGLU's
 *     bf16(g * sigmoid(g)) is a function of the bf16 gate alone, and on all
 *     65,536 gate values it equals the reference's with the host's libm
 *     expf (checked exhaustively on the device, clamp limit 10).
 *
 * BUFFERS. Discrete HBM, no zero-copy: host-pointer entry points copy x in
 * and y out on every call and keep weights resident only for REGISTERED
 * regions (uploaded once at registration, looked up by host range like
 * c/backend_gmetal.mm:240-251). Unregistered weights are uploaded per op.
 * The *_dev entry points take device pointers and a hipStream_t and are
 * asynchronous; the expert store keeps whole expert slabs resident in HBM.
 *
 * THREADING. Host-pointer entry points are synchronous (one stream, waited
 * on before return) and compute-thread only, as the Metal backend
 * (c/backend_gmetal.h:97-99). *_dev calls are stream-ordered; calls that
 * share an expert store's decode workspace must not overlap in time.
 *
 * ENV KNOBS (read once at apus_ghip_enable, like c/backend_gmetal.mm:437-453):
 *   APUS_GHIP_MIN_KB      BF16 hook floor: weights below it stay on the CPU
 *                         (default 0 = offload all).
 *   APUS_GHIP_FP8_MIN_KB  FP8 hook floor (default 0).
 *   APUS_GHIP_MAX_M       activation rows above it stay on the CPU
 *                         (default 0 = unlimited).
 *   APUS_GHIP_DEVICE      HIP device ordinal (default 0).
 */
#ifndef APUS_BACKEND_HIP_H
#define APUS_BACKEND_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================================================================== */
/* 1. Mirror of c/backend_gmetal.h                                           */
/* ======================================================================== */

/* Hook table — replaces ApusGmetalHooks (c/backend_gmetal.h:120-126); same
 * two signatures byte for byte. 0 = produced the result; nonzero = declined
 * (the caller runs its CPU kernel). Shapes: w/codes [O,K] row-major, scales
 * [ceil(O/128)*ceil(K/128)] F32, x [M,K] and y [M,O] BF16 codes. */
typedef struct {
    int (*bf16_gemm)(const uint16_t *w, const uint16_t *x, uint16_t *y,
                     size_t M, size_t O, size_t K);
    int (*fp8blk_linear)(const uint8_t *codes, const float *scales,
                         const uint16_t *x, uint16_t *y,
                         size_t M, size_t O, size_t K);
} ApusGhipHooks;

/* replaces `extern ApusGmetalHooks apus_gmetal_hooks;` (c/backend_gmetal.h:128).
 * The library carries a weak definition so a standalone process links; an
 * engine TU that defines the table (as c/bf16.h:162 does for Metal) wins. */
extern ApusGhipHooks apus_ghip_hooks;

/* replaces apus_gmetal_enable / _disable / _is_enabled
 * (c/backend_gmetal.h:134-137). enable: select the device, create the
 * backend stream, read the env floors, fill the hooks. 0 = ok; nonzero with
 * err filled when no usable gfx950 device is present. Idempotent. */
int  apus_ghip_enable(char *err, size_t errcap);
void apus_ghip_disable(void);
int  apus_ghip_is_enabled(void);

/* replaces apus_gmetal_register_region / _unregister_region
 * (c/backend_gmetal.h:147-148): upload a MODEL-OWNED weight region to HBM
 * once; later ops whose weight range lies inside it use the device mirror.
 * 0 = ok, nonzero = not registered (ops fall back to per-op uploads).
 * Idempotent per pointer; the caller unregisters before freeing. */
int  apus_ghip_register_region(const void *ptr, size_t len);
void apus_ghip_unregister_region(const void *ptr);

/* replaces the counters of c/backend_gmetal.h:153-157. bytes_wrapped =
 * per-op weight uploads (no zero-copy on discrete HBM), bytes_pinned =
 * registered device-mirror bytes. Plus the host<->device copy totals. */
uint64_t apus_ghip_bytes_wrapped(void);
uint64_t apus_ghip_bytes_pinned(void);
uint64_t apus_ghip_dispatches(void);
uint64_t apus_ghip_offload_bf16(void);
uint64_t apus_ghip_offload_fp8blk(void);
uint64_t apus_ghip_bytes_h2d(void);
uint64_t apus_ghip_bytes_d2h(void);

/* replaces apus_gmetal_bf16_gemm / apus_gmetal_fp8blk_linear
 * (c/backend_gmetal.h:162-166): direct entry points, no floors, lazy init.
 * 0 = ok, 1 = no device / unsupported / failure. */
int apus_ghip_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                        size_t M, size_t O, size_t K);
int apus_ghip_fp8blk_linear(const uint8_t *codes, const float *scales,
                            const uint16_t *x, uint16_t *y,
                            size_t M, size_t O, size_t K);

/* Last error message of the calling process ("" when none). */
const char *apus_ghip_last_error(void);

/* ======================================================================== */
/* 2. Extensions (no Metal counterpart)                                      */
/* ======================================================================== */

/* FP8-block dequant to BF16 on the device (K1). Replaces the CPU
 * apus_fp8blk_dequant / _mt (c/fp8blk.h:115-136, 277-317) for callers that
 * want BF16 weights (e.g. dequant-on-fill, c/gcache.h:413-426). Host
 * pointers, synchronous. Bitwise equal to the CPU result. */
int apus_ghip_fp8blk_dequant(const uint8_t *codes, const float *scales,
                             uint16_t *out, size_t O, size_t K);

/* Device-pointer variants (asynchronous on `stream`, a hipStream_t; NULL =
 * the null stream). exact: 0 = fast decode (caller guarantees no 0x7F/0xFF
 * code), 1 = exact integer decode, -1 = scan the codes first and pick.
 * These share process-wide device state: the NaN-scan flag (exact = -1),
 * the exact-decode flag word and the split-K partial buffer of the GEMM
 * path (M >= 16). Calls must therefore not overlap in time: issue them on
 * one stream, and do not run them concurrently with the host-pointer
 * entry points (which use the backend's own stream).
 * Alignment: the GEMM path (M >= 16; weights read once) needs 16-byte
 * aligned codes, x and y, N % 256 == 0 and K % 128 == 0; otherwise the
 * rows go to the streaming GEMV in groups of <= 4, which re-reads the
 * weights ceil(M / 4) times (same results within the tolerance, slower). */
int apus_ghip_fp8blk_dequant_dev(const uint8_t *codes, const float *scales,
                                 uint16_t *out, size_t O, size_t K,
                                 int exact, void *stream);
int apus_ghip_fp8blk_linear_dev(const uint8_t *codes, const float *scales,
                                const uint16_t *x, uint16_t *y,
                                size_t M, size_t O, size_t K,
                                int exact, void *stream);
int apus_ghip_bf16_gemm_dev(const uint16_t *w, const uint16_t *x,
                            uint16_t *y, size_t M, size_t O, size_t K,
                            void *stream);

/* --- HBM-resident expert slab store (replaces the ApusGcacheW views of
 * c/gcache.h:592-643 behind the expert seam c/gmodel.h:1155-1178). One
 * device arena holds every expert's FP8 slab in the reference member order
 * gate.w | gate.s | up.w | up.s | down.w | down.s (c/gcache.h:852-861):
 * 2*(inter*dim + nb) + dim*inter + nb bytes per slab, nb = F32 scale bytes;
 * 25,171,968 B at dim 4096 / inter 2048. Slabs stay FP8 in HBM; kernels
 * dequantize on the fly (bit-exact). */
typedef struct ApusGhipStore ApusGhipStore;

/* Allocate the arena for n_experts slabs (+ the decode workspace). limit =
 * swiglu_limit (10 for GLM-5.3-Flash, reference/config.json:253). */
int apus_ghip_store_open(ApusGhipStore **out, int n_experts, size_t dim,
                         size_t inter, float limit, char *err, size_t errcap);
void apus_ghip_store_close(ApusGhipStore *s);
size_t apus_ghip_store_slab_bytes(const ApusGhipStore *s);
/* One H2D copy of one slab (the reference's one pread per slab). Scans the
 * codes for NaN codes and records the decode path for the expert. */
int apus_ghip_store_put(ApusGhipStore *s, int expert, const void *slab,
                        size_t nbytes);
/* Fill every slab with the deterministic synthetic generator
 * (include/apus_synth.h; bank id selects the streams): codes on device,
 * scales log-uniform in [scale_lo, scale_hi] from the host. */
int apus_ghip_store_synth(ApusGhipStore *s, uint64_t seed, int bank,
                          float scale_lo, float scale_hi);
/* Device address of expert e's slab (NULL when out of range): members in
 * the same order at 256-byte aligned offsets. */
const void *apus_ghip_store_slab_dev(const ApusGhipStore *s, int expert);
/* The layer's shared expert (c/gmoe.h:325-336; every token runs it and its
 * output is added last, with one more bf16 rounding and no weight: out =
 * bf16(routed + shared)). The slab has the routed experts' layout and
 * intermediate size (n_shared_experts = 1 makes the shared intermediate
 * moe_intermediate_size, c/gmodel.h:963-964); one H2D copy into a slot the
 * store reserves after the routed experts. Once set, apus_ghip_moe_decode*
 * and apus_ghip_moe_prefill* include it; slab NULL removes it. The decode
 * with a shared expert needs inter <= 8 x the device's CUs (2048 on 256
 * CUs). Extension: the reference dequantizes the shared expert at open
 * and runs it on the CPU. */
int apus_ghip_store_put_shared(ApusGhipStore *s, const void *slab, size_t nbytes);
/* Read expert e's slab back in the host slab format (row-major members,
 * c/gcache.h:852-861 order): the inverse of apus_ghip_store_put.
 * Extension; no counterpart in the reference. */
int apus_ghip_store_get(ApusGhipStore *s, int expert, void *slab,
                        size_t nbytes);
/* Fill the store from a converted v2 container directory (the format the
 * reference's expert cache opens, c/gcache.h:832-930; schema
 * tests/m1/README.md:21-55): parses <dir>/apus.index.json (format_version
 * 2, model_type glm5_next), takes the expert_slabs records of block
 * "layers.<layer>" (each must hold exactly one slab), and loads every
 * listed expert with one pread of its slab from <dir>/<shard> at the
 * record's offset (c/gcache.h:394-451) into pinned staging and one H2D
 * copy, overlapping the next read. Unlisted experts are left as they are.
 * n_loaded: experts loaded (may be NULL). 0 = ok, else err filled. */
int apus_ghip_store_load_container(ApusGhipStore *s, const char *dir, int layer,
                                   int *n_loaded, char *err, size_t errcap);
/* The index lookup alone (host only, no device): shard file name and file
 * offset of the slab (layers.<layer>, expert), checked to hold slab_bytes.
 * Extension for loaders and tests; no counterpart in the reference. */
int apus_ghip_container_slab(const char *dir, int layer, int expert, size_t slab_bytes,
                             char *shard, size_t shard_cap, uint64_t *offset,
                             char *err, size_t errcap);
/* Dequant-on-fill: expert e's BF16 payload [gate | up | down] into a host
 * buffer (3*inter*dim u16), bitwise c/gcache.h:413-426. */
int apus_ghip_store_expert_bf16(ApusGhipStore *s, int expert,
                                uint16_t *payload);

/* --- MoE router with the reference semantics (apus_gmoe_router,
 * c/gmoe.h:191-208; numerics c/gmhc.h:157-185), on device pointers:
 * gate logits = gate_w [E, dim] bf16 . x [dim] bf16 in f32 (a GEMV: the
 * same tolerance class as every GEMV here; pass logits [E] f32 instead,
 * with gate_w / x NULL, to start from given logits), scores = numpy-stable
 * sigmoid, selection = stable top-k (ties -> lower id) of score + gate_bias
 * (the bias selects, it never weighs), w = the selected scores / (numpy
 * pairwise sum + 1e-20) * route_scale. Outputs idx / w [topk] in selection
 * order (as the reference) and, when scores is non-NULL, scores [E]; the
 * result feeds apus_ghip_moe_decode_dev / _prefill_dev as idx / w.
 * E <= 512, topk <= 16, dim % 8 == 0. One kernel launch, asynchronous on
 * `stream`; the gate-logit form uses a process-wide device workspace, so
 * calls that overlap on the device race (order them on one stream). 0 = ok. */
int apus_ghip_moe_router_dev(const uint16_t *x, const uint16_t *gate_w,
                             const float *logits, const float *gate_bias, int E,
                             size_t dim, int topk, float route_scale, float *scores,
                             int32_t *idx, float *w, void *stream);

/* --- routed MoE decode (one token): SwiGLU experts + ordered combine,
 * c/gmoe.h:210-227 + 307-320 (+ 325-336 when the store holds a shared
 * expert, apus_ghip_store_put_shared), without the router. One
 * persistent launch (one workgroup per CU, all resident at once): routing,
 * gate/up GEMVs with the SwiGLU epilogue (activations to HBM, two per word,
 * into a buffer that holds only a sentinel until the launch writes it),
 * then down GEMVs, each wave starting as soon as its expert's activations
 * are all in, and the ascending-expert bf16-per-add combine. Calls that
 * share a store must not overlap in time (one stream). Each call flips a
 * host-side parity that picks which of two activation buffers it writes
 * (it refills the other for the next call) and advances a host-side tag,
 * so the device variant cannot be captured into a graph (a replay would
 * reuse the recorded buffer): it returns 1 on a capturing stream and
 * launches nothing.
 * Routing either given (idx/w [topk]) or computed on the device from
 * logits [n_experts] f32: stable top-k (ties -> lower id), w = softmax over
 * the k selected logits. Host-pointer variant is synchronous. */
int apus_ghip_moe_decode(ApusGhipStore *s, const uint16_t *x,
                         const int32_t *idx, const float *w, int topk,
                         uint16_t *out);
int apus_ghip_moe_decode_dev(ApusGhipStore *s, const uint16_t *x,
                             const float *logits, const int32_t *idx,
                             const float *w, int topk, uint16_t *out,
                             void *stream);

/* --- the engine's decode step in one launch: the reference router
 * (apus_gmoe_router, c/gmoe.h:191-208: gate logits gate_w [E, dim] bf16 .
 * x in f32, numpy-stable sigmoid scores, stable top-k of score + gate_bias
 * -- the bias selects, it never weighs -- and w = the selected scores over
 * their numpy pairwise sum + 1e-20, times route_scale) feeding the routed
 * experts and the ascending-expert combine (c/gmoe.h:294-320), and the
 * shared expert when the store holds one (c/gmoe.h:325-336). Replaces
 * apus_ghip_moe_router_dev followed by apus_ghip_moe_decode_dev (the same
 * logits, picks, weights and outputs, bitwise) with one launch: the
 * workgroups compute the gate logits, hand them over as words tagged with
 * the launch, and each selects for itself. idx_out / w_out (device [topk],
 * both or neither): the picks in selection order. E <= 512 and E <= 8 x the
 * device's CUs; 16-byte aligned x and gate_w. Stream-ordered, the same
 * no-overlap and no-capture rules as apus_ghip_moe_decode_dev; device-side
 * failures go to apus_ghip_store_status. No counterpart in the Metal
 * backend. */
int apus_ghip_moe_decode_router_dev(ApusGhipStore *s, const uint16_t *x,
                                    const uint16_t *gate_w, const float *gate_bias,
                                    float route_scale, int topk, uint16_t *out,
                                    int32_t *idx_out, float *w_out, void *stream);

/* --- routed MoE prefill (T tokens): the reference runs, per token, the
 * selected experts and the ordered combine (c/gmoe.h:278-320, expert body
 * c/gmoe.h:210-227); here the same result is computed as grouped GEMMs over
 * expert-sorted (token, expert) pairs: a GPU stable counting sort of the
 * pairs, one gate/up GEMM launch with the SwiGLU epilogue and one down GEMM
 * launch over all experts (FP8 tiles dequantized bit-exactly in registers,
 * BF16 MFMA, fp32 accumulation), then the ascending-expert bf16-per-add
 * combine. idx/w [T, topk] row-major (token t's slots at t*topk). A repeated
 * id inside one token counts once, with its first slot's weight, as the
 * reference loop. Needs dim % 256 == 0, inter % 128 == 0, <= 1024 experts,
 * topk <= 16. Tolerance class as the GEMV (floor = sum_e |contrib_e|).
 * The device variant is stream-ordered; ids out of range are dropped from
 * the sum (the host variant rejects them before launching). All prefill
 * calls share one process-wide workspace (grown on demand; reserve to size
 * it up front), so calls on different streams must not overlap in time. */
int apus_ghip_moe_prefill_reserve(const ApusGhipStore *s, size_t tokens,
                                  int topk);
int apus_ghip_moe_prefill(ApusGhipStore *s, const uint16_t *x, size_t T,
                          const int32_t *idx, const float *w, int topk,
                          uint16_t *out);
int apus_ghip_moe_prefill_dev(ApusGhipStore *s, const uint16_t *x, size_t T,
                              const int32_t *idx, const float *w, int topk,
                              uint16_t *out, void *stream);

/* Device-side failures of the asynchronous MoE entries. No counterpart in
 * the reference: its backend ops are synchronous and return the failure
 * themselves (c/backend_gmetal.h:111-119), which the host-pointer entries
 * here still do. A *_dev call returns 0 once its launch is queued; what
 * goes wrong on the device afterwards is ORed into the store's sticky
 * error word: 2 = an expert id outside 0..n_experts-1 was dropped (decode
 * or prefill; that pair is missing from the sum), 4 = a decode's gate/up
 * -> down hand-off wait ran out (another kernel held CUs the launch
 * needed; the output of that decode is invalid). Waits for `stream` (a
 * hipStream_t, NULL = the null stream), stores the word in *code and,
 * with clear != 0, resets it. The host-pointer decode and prefill reset
 * the word before their own launch, so read a *_dev call's status before
 * the next host-pointer MoE call on the store. Synchronous; not for
 * streams under graph capture. 0 = the word was read. */
int apus_ghip_store_status(ApusGhipStore *s, void *stream, int clear,
                           uint32_t *code);

/* Allocation-free variant of apus_ghip_moe_prefill_dev. No counterpart in
 * the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels and results (bitwise) as
 * apus_ghip_moe_prefill_dev, but the workspace (header and queue counters,
 * tile list, pair permutation, the H and O pair rows) lives in a fixed
 * 32 MiB device array of the library instead of the grow-on-demand
 * workspace: it calls no hipMalloc / hipFree and no allocating library
 * routine. The call's workspace must fit that array: at dim 4096, inter
 * 2048, 288 experts that is T * topk <= ~2600 pairs (T <= ~320 tokens at
 * top-8); larger calls return 1 with the needed size in
 * apus_ghip_last_error. Needs the library initialised (apus_ghip_enable or
 * apus_ghip_store_open first). Every call on a GPU shares that GPU's array
 * (the per-call counters are cleared by each call's own fill kernel), so
 * calls that overlap in time on one GPU race: order them on one stream. */
int apus_ghip_moe_prefill_dev_noalloc(ApusGhipStore *s, const uint16_t *x, size_t T,
                                      const int32_t *idx, const float *w, int topk,
                                      uint16_t *out, void *stream);

/* --- timing (no reference counterpart; for benchmarks and profilers).
 * events: n caller-created hipEvent_t handles, NULL/0 turns it off. While
 * set, launches carry start/stop events in their dispatch packets
 * (hipExtLaunchKernelGGL), so an event pair spans exactly one kernel:
 * apus_ghip_moe_decode_dev (n >= 2) records events[0] and events[1]
 * around its one launch;
 * apus_ghip_fp8blk_linear_dev, apus_ghip_bf16_gemm_dev and
 * apus_ghip_moe_router_dev (n >= 2) start events[0] with their first launch
 * and stop events[1] with their last; apus_ghip_moe_prefill_dev
 * (n >= 8) times the permutation with events[0..1], the gate/up GEMM with
 * events[2..3], the down GEMM with events[4..5] and the combine with
 * events[6..7]. Process-wide, not
 * thread-safe; the events must outlive their use. */
void apus_ghip_set_trace_events(void *const *events, int n);

/* Hold `stream` for `us` microseconds (<= 1 s) with one wave that waits on
 * the wall clock and touches no memory; asynchronous. A benchmark enqueues
 * it before a timed region's start event so the host has queued the timed
 * steps before the device reaches them. No reference counterpart. 0 = ok. */
int apus_ghip_stream_hold(void *stream, uint32_t us);

#ifdef __cplusplus
}
#endif
#endif /* APUS_BACKEND_HIP_H */
