/*
 * ghip_internal.h — launchers exported by the .hip kernel units to the C
 * host layer (ghip_backend.c). Plain C ABI: device pointers, sizes and a
 * hipStream_t. Every launcher validates the shape it is given against what
 * its kernel and grid assume and returns a hipError_t (hipErrorInvalidValue
 * for a shape the kernel cannot take) without launching anything invalid.
 */
#ifndef GHIP_INTERNAL_H
#define GHIP_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* K1: out[O,K] bf16 = bf16(e4m3(codes) * scale of the 128x128 block).
 * exact != 0 selects the integer decode (required for NaN codes). */
hipError_t ghip_launch_dequant(const uint8_t *codes, const float *scales,
                               uint16_t *out, size_t O, size_t K, int exact,
                               hipStream_t st);

/* Scan codes for the NaN codes 0x7F/0xFF: *flag (device u32) |= 1 when any
 * is present. The caller zeroes *flag first. */
hipError_t ghip_launch_nan_scan(const uint8_t *codes, size_t n,
                                uint32_t *flag, hipStream_t st);

/* K2: y[M,O] bf16 = x[M,K] . dequant(W)^T, fp32 accumulate, RNE narrow.
 * exact_dev: device u32 flag (nonzero -> exact decode); may be NULL (fast).
 * Any M >= 1, any O, K >= 1. */
hipError_t ghip_launch_fp8_linear(const uint8_t *codes, const float *scales,
                                  const uint16_t *x, uint16_t *y, size_t M,
                                  size_t O, size_t K, const uint32_t *exact_dev,
                                  const hipEvent_t *ev, hipStream_t st);

/* BF16-weight GEMV/GEMM: y[M,O] = x[M,K] . W[O,K]^T. Any shape. ev: NULL or
 * two timing events (start on the first launch, stop on the last). */
hipError_t ghip_launch_bf16_linear(const uint16_t *w, const uint16_t *x,
                                   uint16_t *y, size_t M, size_t O, size_t K,
                                   const hipEvent_t *ev, hipStream_t st);

/* K3 MoE decode workspace: the SwiGLU activations h handed from the
 * gate/up phase to the down phase as words of two bf16 values (the even
 * row in bits 0..15), in two buffers that alternate between launches: the
 * one a launch writes holds only the sentinel 0xffffffff when it starts,
 * and it refills the other (both filled at creation); an error word, the
 * host's current tag (the router's logit words) and buffer parity. */
typedef struct {
    uint32_t *hw;         /* device [2][17 slots][hw_inter / 2] u32: 16 routed + the shared
                             expert, per buffer */
    uint32_t hw_inter;    /* inter the words were sized for */
    uint32_t *err;        /* device u32: 2 = invalid expert id, 4 = hand-off wait ran out */
    uint64_t *lw;         /* device [512] u64: the router-fed decode's tagged gate logits
                             (the launch's tag in bits 32..47, the f32 logit in 0..31) */
    uint32_t n_cu;        /* grid: one workgroup per CU */
    uint32_t tag;         /* host: the last launch's tag (0 before the first) */
    uint32_t hpar;        /* host: the h buffer the next launch writes (0 or 1) */
} GhipMoeDecodeWs;

/* The reference router's inputs for the router-fed decode (c/gmoe.h:191-208):
 * gate_w [E, dim] bf16 (16-byte aligned), bias [E] f32 (selection only),
 * route_scale; idx_out / w_out [topk] (both or neither) receive the picks. */
typedef struct {
    const uint16_t *gate_w;
    const float *bias;
    float route_scale;
    int32_t *idx_out;
    float *w_out;
} GhipRouterArgs;

/* Streaming GEMV set-up (dynamic-LDS limits, persistent grid bound). */
hipError_t ghip_linear_init(uint32_t n_cu);

/* Raise the decode kernel's dynamic-LDS limit (once per process). */
hipError_t ghip_moe_decode_init(void);

/* Expert bank view for the kernels: slab s of expert e at base + e*stride;
 * member byte offsets inside a slab (c/gcache.h:852-861 order). */
typedef struct {
    const uint8_t *base;
    size_t stride;               /* bytes between consecutive slabs */
    size_t off_gw, off_gs, off_uw, off_us, off_dw, off_ds;
    uint32_t n_experts, dim, inter;
    const uint32_t *nan_flags;   /* device [n_experts] u32 (required by decode) or NULL */
    uint32_t *err;               /* device u32, the store's sticky error word (2 = an
                                    invalid expert id was dropped, 4 = a decode hand-off
                                    wait ran out) or NULL */
    uint32_t has_shared;         /* 1: a shared expert's slab at index n_experts (same
                                    layout and inter), added last to every token */
} GhipBank;

/* K3: routed MoE decode for one token (routing, gate/up + SwiGLU, down +
 * ordered combine, + the shared expert when the bank has one) as one launch
 * on st (ws->n_cu workgroups); ev: NULL or 2 events recorded around it. The
 * routing is one of: router (the reference router computed in the launch),
 * logits (device f32 [n_experts]; top-k + softmax on the device) or idx/w
 * (device [topk]). out: device [dim] bf16. Advances ws->tag. Launches that
 * share a workspace must not overlap in time. */
hipError_t ghip_launch_moe_decode(const GhipBank *bank, const uint16_t *x,
                                  const float *logits, const int32_t *idx,
                                  const float *w, const GhipRouterArgs *router,
                                  int topk, float limit,
                                  uint16_t *out, GhipMoeDecodeWs *ws,
                                  const hipEvent_t *ev, hipStream_t st);

/* Router with the reference semantics (c/gmoe.h:191-208): gate logits (a
 * GEMV over gate_w [E, dim] bf16 into logits_ws [E] f32, or given
 * logits_in), numpy-stable sigmoid scores, stable top-k of score + bias,
 * pairwise-sum normalization x scale. scores [E] optional; idx / w [topk]
 * in selection order. E <= 512, topk <= 16. One launch either way; with
 * gate_w, `count` is a device word that is 0 before the launch and 0 after
 * it (launches that overlap on one device race on it and on logits_ws).
 * ev: NULL or two timing events around the launch. */
hipError_t ghip_launch_moe_router(const uint16_t *x, const uint16_t *gate_w,
                                  const float *logits_in, float *logits_ws,
                                  uint32_t *count, const float *bias, uint32_t E,
                                  uint32_t dim, int topk, float scale, float *scores,
                                  int32_t *idx, float *w, const hipEvent_t *ev,
                                  hipStream_t st);

/* K4 prefill workspace (device; sized for cap_pairs = T * topk pairs). */
#define PF_HDR_NTILES 0
#define PF_HDR_NPAIRS 1
#define PF_HDR_ERR 2
#define PF_HDR_Q 16           /* 2 x 8 item-queue counters (GEMM, XCD) */
#define PF_HDR_WORDS 32
typedef struct {
    uint32_t *hdr;        /* PF_HDR_WORDS u32: tiles, kept pairs, error,
                             the GEMMs' per-XCD item counters; zeroed per call */
    uint32_t *cnt;        /* [chunks, n_experts] histograms -> offsets */
    uint32_t *tiles;      /* [max_tiles] x {expert, row0, rows, 0} */
    int32_t *eid;         /* [pairs] expert of a kept pair, else -1 */
    int32_t *perm;        /* [pairs] sorted row -> pair */
    int32_t *pos;         /* [pairs] pair -> sorted row, -1 if dropped */
    uint16_t *h;          /* [pairs, inter] bf16 SwiGLU activations */
    uint16_t *o;          /* [pairs, dim] bf16 expert outputs */
    size_t cap_pairs;
    uint32_t n_cu;        /* persistent GEMM grid: the device's CU count */
} GhipMoePrefillWs;

size_t ghip_moe_prefill_max_tiles(size_t pairs, uint32_t n_experts);
size_t ghip_moe_prefill_chunks(size_t pairs);
/* Raise the GEMM kernels' dynamic-LDS limit (once per process). */
hipError_t ghip_moe_prefill_init(void);

/* Allocation-free prefill workspace: a fixed device array of
 * GHIP_PF_SCRATCH_BYTES per GPU. ghip_pf_scratch_init (once per device, that
 * device current) takes its device address; ghip_pf_scratch_need is the
 * bytes a call needs; ghip_pf_scratch_ws carves the workspace of one call
 * out of it (hipErrorOutOfMemory when it does not fit, hipErrorNotInitialized
 * before init). */
#define GHIP_PF_SCRATCH_BYTES ((size_t)32 << 20)
#define GHIP_MAX_DEVICES 64
hipError_t ghip_pf_scratch_init(int device);
size_t ghip_pf_scratch_need(size_t pairs, uint32_t n_experts, uint32_t dim,
                            uint32_t inter);
hipError_t ghip_pf_scratch_ws(int device, size_t pairs, uint32_t n_experts, uint32_t dim,
                              uint32_t inter, uint32_t n_cu, GhipMoePrefillWs *ws);

/* K4: routed MoE prefill for T tokens: permutation, grouped gate/up GEMM
 * with the SwiGLU epilogue, grouped down GEMM, ordered combine (stream
 * ordered on st). x [T, dim], idx/w [T, topk], out [T, dim], all device.
 * ev: NULL or 8 events (permutation, gate/up, down, combine start/stop). */
hipError_t ghip_launch_moe_prefill(const GhipBank *bank, const uint16_t *x,
                                   size_t T, const int32_t *idx, const float *w,
                                   int topk, float limit, uint16_t *out,
                                   const GhipMoePrefillWs *ws,
                                   const hipEvent_t *ev, hipStream_t st);

/* Dense FP8-block GEMM on MFMA (the prefill tile body): Y [M, N] =
 * bf16(X [M, K] . dequant(W [N, K])^T). Shapes it takes: N % 256 == 0,
 * K % 128 == 0, K <= 16384, 16-byte aligned codes, X and Y
 * (ghip_fp8_gemm_fits). Persistent grid of at most n_cu workgroups; the
 * dynamic-LDS limit is raised by ghip_moe_prefill_init. ev: NULL or 2
 * events. */
int ghip_fp8_gemm_fits(size_t M, size_t N, size_t K, const void *codes, const void *x,
                       const void *y);
hipError_t ghip_launch_fp8_gemm(const uint8_t *codes, const float *scales,
                                const uint16_t *x, uint16_t *y, size_t M, size_t N,
                                size_t K, const uint32_t *exact_dev, uint32_t n_cu,
                                const hipEvent_t *ev, hipStream_t st);

/* One expert slab record of a converted v2 container's apus.index.json
 * (c/gcache.h:896-930): the shard file name and the slab's file offset. */
typedef struct {
    int expert;
    char shard[256];
    uint64_t offset, nbytes;
} GhipSlabRec;

/* Parse <dir>/apus.index.json (format_version 2, model_type glm5_next) and
 * return the slab records of block "layers.<layer>" (malloc'd, *n_out of
 * them), each checked to hold exactly slab_bytes. 0 on success, else err. */
int ghip_container_layer(const char *dir, int layer, size_t slab_bytes,
                         GhipSlabRec **out, int *n_out, char *err, size_t errcap);

/* Fill n u32 words with value (a kernel, not a memset, so callers may
 * capture it in a graph). */
hipError_t ghip_launch_fill_u32(uint32_t *p, size_t n, uint32_t value,
                                hipStream_t st);

/* Hold stream st for `ticks` wall-clock ticks (hipDeviceAttributeWallClockRate
 * kHz): one wave that waits and exits, touching no memory. */
hipError_t ghip_launch_hold(uint64_t ticks, hipStream_t st);

/* Device fill of synthetic FP8 codes (same bytes as apus_synth_fp8_codes). */
hipError_t ghip_launch_synth_codes(uint8_t *out, size_t n, uint64_t key,
                                   uint64_t offset, hipStream_t st);
/* Device fill of bf16 N(0,1) through a device copy of the quantile table. */
hipError_t ghip_launch_synth_bf16(uint16_t *out, size_t n, uint64_t key,
                                  uint64_t offset, const uint16_t *table,
                                  hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif /* GHIP_INTERNAL_H */
