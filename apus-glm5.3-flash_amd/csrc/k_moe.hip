/*
 * k_moe.hip — K3: routed-MoE decode for one token (gfx950), three launches
 * on one stream, no inter-workgroup waits:
 *
 *   k_moe_route   one wave: routing -> workspace (nsel, expert ids ascending,
 *                 weights). Either the harness routing on the device (stable
 *                 top-k of f32 logits, ties -> lower id, softmax over the k
 *                 selected) or given idx/w, deduplicated keeping the first
 *                 slot of a repeated id (c/gmoe.h:309-312) and sorted by id.
 *   k_moe_gateup  one workgroup per (slot q, 16 rows): g and u GEMVs over
 *                 dim with the FP8 dequant fused (bit-exact weights), the
 *                 SwiGLU epilogue of c/gmoe.h:217-225 -> h[q] (bf16).
 *   k_moe_down    one workgroup per 16 output rows: wave q computes expert
 *                 q's down GEMV (h[q] . Wd^T, full inter in-wave), then the
 *                 ascending-expert combine y = bf16(y + bf16(bf16(o)*w))
 *                 (c/gmoe.h:307-320) runs in-workgroup — no atomics, no
 *                 cross-workgroup reduction, deterministic.
 *
 * A single persistent launch with completion counters was tried first: its
 * agent-scope release/acquire fences (an L2 write-back / invalidate per wave
 * per tile) cost ~10x the weight streaming, so the phases are split at
 * kernel boundaries, which order the h and routing handoffs for free.
 *
 * GEMV inner loop (ghip_chunk_*, as k_linear.hip): 16 rows per MFMA group,
 * 128-wide k chunks (one scale block, two 16-byte code loads per lane, full
 * 128-byte lines per wave), dequant in registers, x (or h) as the A operand
 * from LDS; weight loads are issued before the activation is staged so the
 * two latencies overlap.
 */
#include "ghip_device.h"
#include "ghip_internal.h"

#define MD_NW 8                  /* waves per workgroup */
#define MD_T 16                  /* rows per tile (one MFMA group) */
#define MD_MAXK 16               /* max routed slots */
#define MD_LOADS 16              /* 16-byte loads in flight per lane */

/* routing workspace (u32 words): [0] nsel, [1..16] ids, [17..32] weights */
#define RT_NSEL 0
#define RT_IDS 1
#define RT_W (1 + MD_MAXK)

/* ------------------------------------------------------------------------ */
/* routing                                                                  */
/* ------------------------------------------------------------------------ */

#define RT_REG 8                 /* logits per lane held in registers */
#define RT_MAXE (64 * RT_REG)    /* 512 experts */

/* Monotone key of (value, index): larger value first, then LOWER index —
 * the stable top-k order of c/gmoe.h:175-189 — as one unsigned 64-bit max. */
__device__ __forceinline__ uint64_t rt_key(float v, int i) {
    /* -0 and +0 compare equal in the reference, so they must share a key */
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
}

__device__ __forceinline__ uint64_t rt_wave_max(uint64_t k) {
    for (int off = 32; off > 0; off >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)k, off, 64);
        uint32_t hi = __shfl_xor((uint32_t)(k >> 32), off, 64);
        uint64_t o = ((uint64_t)hi << 32) | lo;
        k = o > k ? o : k;
    }
    return k;
}

/* One wave. Logits live in registers (RT_REG per lane); each of the k
 * rounds takes the lane-local best key and one 64-bit wave max. */
__global__ __launch_bounds__(64) void k_moe_route(
    const float *__restrict__ logits, const int32_t *__restrict__ idx,
    const float *__restrict__ w, int topk, int E, uint32_t *__restrict__ route,
    uint32_t *__restrict__ err) {
    __shared__ int32_t te[MD_MAXK];
    __shared__ float tw[MD_MAXK];
    const int lane = threadIdx.x;
    if (logits) {
        uint64_t key[RT_REG];
#pragma unroll
        for (int s = 0; s < RT_REG; s++) {
            int i = lane + 64 * s;
            key[s] = i < E ? rt_key(logits[i], i) : 0ull;
        }
        for (int j = 0; j < topk; j++) {
            uint64_t b = 0;
#pragma unroll
            for (int s = 0; s < RT_REG; s++) b = key[s] > b ? key[s] : b;
            b = rt_wave_max(b);
            const int bi = (int)(0xffffffffu - (uint32_t)b);
#pragma unroll
            for (int s = 0; s < RT_REG; s++)
                if (key[s] == b) key[s] = 0ull;
            if (lane == 0) {
                /* the value is in the key: undo the monotone transform */
                const uint32_t hi = (uint32_t)(b >> 32);
                te[j] = bi;
                tw[j] = __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
            }
        }
        if (lane == 0) {
            float m = tw[0], ssum = 0.0f;
            for (int j = 0; j < topk; j++) {
                tw[j] = expf(tw[j] - m);
                ssum = ssum + tw[j];
            }
            for (int j = 0; j < topk; j++) tw[j] = tw[j] / ssum;
        }
    } else if (lane < topk) {
        te[lane] = idx[lane];
        tw[lane] = w[lane];
    }
    __syncthreads();
    /* lane j < topk owns slot j: dropped if its id repeats an earlier slot
     * (first-match slot, c/gmoe.h:309-312) or is out of range; kept slots
     * are placed by ascending expert id (the combine order). */
    const int e = lane < topk ? te[lane] : -1;
    const float wj = lane < topk ? tw[lane] : 0.0f;
    bool keep = lane < topk;
    if (keep && (e < 0 || e >= E)) { keep = false; atomicOr(err, 2u); }
    for (int q = 0; q < MD_MAXK; q++) {
        const int eq = __shfl(e, q, 64);
        if (q < lane && q < topk && eq == e) keep = false;
    }
    int pos = 0;
    for (int q = 0; q < MD_MAXK; q++) {
        const int eq = __shfl(e, q, 64);
        const int kq = __shfl((int)keep, q, 64);
        pos += (kq && eq < e);
    }
    const uint64_t kept = __ballot(keep);
    if (keep) {
        route[RT_IDS + pos] = (uint32_t)e;
        route[RT_W + pos] = __float_as_uint(wj);
    }
    const uint32_t nsel = (uint32_t)__popcll(kept);
    if (lane == 0) route[RT_NSEL] = nsel;
    if (lane >= (int)nsel && lane < MD_MAXK) {
        route[RT_IDS + lane] = 0u;
        route[RT_W + lane] = 0u;
    }
}

/* ------------------------------------------------------------------------ */
/* gate/up + SwiGLU                                                         */
/* ------------------------------------------------------------------------ */

#define GU_U 4                   /* chunks per matrix per batch (16 loads) */

/* buf / scg / scu hold the first batch on entry (issued before x was
 * staged) and are refilled in place, so one set of registers streams. */
template <bool EXACT>
__device__ __forceinline__ void gateup_tile(const uint8_t *wg, const uint8_t *wu,
                                            const float *sg, const float *su,
                                            const uint16_t *xa, uint32_t nch,
                                            uint32_t wv, ghip_chunk (&buf)[2 * GU_U],
                                            float (&scg)[GU_U], float (&scu)[GU_U],
                                            ghip_f32x4 &ag, ghip_f32x4 &au) {
    for (uint32_t c0 = wv; c0 < nch; c0 += MD_NW * GU_U) {
        if (c0 != wv) {
#pragma unroll
            for (int u = 0; u < GU_U; u++) {
                uint32_t c = min(c0 + u * MD_NW, nch - 1u);
                buf[2 * u] = ghip_chunk_load(wg + (size_t)c * 128);
                buf[2 * u + 1] = ghip_chunk_load(wu + (size_t)c * 128);
                scg[u] = sg[c];
                scu[u] = su[c];
            }
        }
#pragma unroll
        for (int u = 0; u < GU_U; u++) {
            uint32_t c = c0 + u * MD_NW;
            if (c < nch) {
                ghip_chunk_mfma<EXACT>(buf[2 * u], scg[u], xa + c * 128, ag);
                ghip_chunk_mfma<EXACT>(buf[2 * u + 1], scu[u], xa + c * 128, au);
            }
        }
    }
}

__global__ __launch_bounds__(MD_NW * 64, 2) void k_moe_gateup(
    GhipBank bank, const uint16_t *__restrict__ x, const uint32_t *__restrict__ route,
    float limit, uint16_t *__restrict__ h) {
    extern __shared__ __align__(16) uint16_t xs[];      /* x [dim] */
    __shared__ float red[2][MD_NW][16];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t dim = bank.dim, inter = bank.inter;
    const uint32_t tiles = inter / MD_T;
    const uint32_t q = blockIdx.x / tiles, r0 = (blockIdx.x - q * tiles) * MD_T;
    const uint32_t nsel = __builtin_amdgcn_readfirstlane(route[RT_NSEL]);
    if (q >= nsel) return;
    const uint32_t e = __builtin_amdgcn_readfirstlane(route[RT_IDS + q]);
    const uint8_t *slab = bank.base + (size_t)e * bank.stride;
    const bool exact = bank.nan_flags && bank.nan_flags[e];
    const uint8_t *wg = slab + bank.off_gw + (size_t)(r0 + n) * dim + 32u * g;
    const uint8_t *wu = slab + bank.off_uw + (size_t)(r0 + n) * dim + 32u * g;
    const uint32_t nkb = dim >> 7;
    const float *sg = (const float *)(slab + bank.off_gs) + (size_t)(r0 >> 7) * nkb;
    const float *su = (const float *)(slab + bank.off_us) + (size_t)(r0 >> 7) * nkb;
    const uint32_t nch = dim >> 7;
    /* this wave's x slices first, then the first batch of weights, then
     * the slices into LDS (wave-local: no workgroup barrier) */
    ghip_stage stx;
    ghip_wstage_load(stx, x, 1u, dim, nch, wv, MD_NW, lane);
    ghip_chunk pre[2 * GU_U];
    float scg[GU_U], scu[GU_U];
#pragma unroll
    for (int u = 0; u < GU_U; u++) {
        uint32_t c = min(wv + u * MD_NW, nch - 1u);     /* unconditional */
        pre[2 * u] = ghip_chunk_load(wg + (size_t)c * 128);
        pre[2 * u + 1] = ghip_chunk_load(wu + (size_t)c * 128);
        scg[u] = sg[c];
        scu[u] = su[c];
    }
    ghip_wstage_store(stx, xs, x, 1u, dim, nch, wv, MD_NW, lane);
    ghip_f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    if (exact) gateup_tile<true>(wg, wu, sg, su, xs + 32u * g, nch, wv, pre, scg, scu, ag, au);
    else gateup_tile<false>(wg, wu, sg, su, xs + 32u * g, nch, wv, pre, scg, scu, ag, au);
    if (g == 0) { red[0][wv][n] = ag[0]; red[1][wv][n] = au[0]; }
    __syncthreads();
    if (tid < 16) {
        float gs = 0.0f, us = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < MD_NW; w2++) { gs += red[0][w2][tid]; us += red[1][w2][tid]; }
        h[(size_t)q * inter + r0 + tid] =
            (uint16_t)ghip_swiglu(ghip_bf16_round(gs), ghip_bf16_round(us), limit);
    }
}

/* ------------------------------------------------------------------------ */
/* down + ordered combine                                                   */
/* ------------------------------------------------------------------------ */

#define DN_U 8                   /* chunks in flight per lane (16 loads) */

/* buf / sc hold the first DN_U chunks on entry and are refilled in place. */
template <bool EXACT>
__device__ __forceinline__ ghip_f32x4 down_rows(const uint8_t *wr, const float *srow,
                                                const uint16_t *ha, uint32_t nch,
                                                ghip_chunk (&buf)[DN_U],
                                                float (&sc)[DN_U]) {
    ghip_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c0 = 0; c0 < nch; c0 += DN_U) {
        if (c0 != 0) {
#pragma unroll
            for (int u = 0; u < DN_U; u++) {
                uint32_t c = min(c0 + u, nch - 1u);
                buf[u] = ghip_chunk_load(wr + (size_t)c * 128);
                sc[u] = srow[c];
            }
        }
#pragma unroll
        for (int u = 0; u < DN_U; u++) {
            uint32_t c = c0 + u;
            if (c < nch) ghip_chunk_mfma<EXACT>(buf[u], sc[u], ha + c * 128, acc);
        }
    }
    return acc;
}

__global__ __launch_bounds__(MD_NW * 64, 2) void k_moe_down(
    GhipBank bank, const uint16_t *__restrict__ h, const uint32_t *__restrict__ route,
    uint16_t *__restrict__ out) {
    extern __shared__ __align__(16) uint16_t hs[];      /* h [nsel][inter] */
    __shared__ float oq[MD_MAXK][16];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t inter = bank.inter;
    const uint32_t r0 = blockIdx.x * MD_T;
    const uint32_t nsel = __builtin_amdgcn_readfirstlane(route[RT_NSEL]);
    const uint32_t nch = inter >> 7;
    const uint32_t nkb = inter >> 7;
    /* this wave's h[q] first (wave-local), then its weights, then h[q]
     * into LDS; a wave holds one expert's full K */
    const uint32_t q0 = wv < nsel ? wv : 0u;
    ghip_stage sth;
    ghip_wstage_load(sth, h + (size_t)q0 * inter, 1u, inter, nch, 0u, 1u, lane);
    ghip_chunk pre[DN_U];
    float sc[DN_U];
    {
        /* unconditional (a wave without a slot reloads slot 0's rows and
         * discards them) so the waitcnt pass sees a fixed load count */
        const uint32_t e = __builtin_amdgcn_readfirstlane(
            route[RT_IDS + (wv < nsel ? wv : 0u)]);
        const uint8_t *slab = bank.base + (size_t)e * bank.stride;
        const uint8_t *wr0 = slab + bank.off_dw + (size_t)(r0 + n) * inter + 32u * g;
        const float *sr0 = (const float *)(slab + bank.off_ds) + (size_t)(r0 >> 7) * nkb;
#pragma unroll
        for (int u = 0; u < DN_U; u++) {
            const uint32_t c = min((uint32_t)u, nch - 1u);
            pre[u] = ghip_chunk_load(wr0 + (size_t)c * 128);
            sc[u] = sr0[c];
        }
    }
    ghip_wstage_store(sth, hs + (size_t)q0 * inter, h + (size_t)q0 * inter, 1u, inter,
                      nch, 0u, 1u, lane);
    for (uint32_t q = wv; q < nsel; q += MD_NW) {
        const uint32_t e = __builtin_amdgcn_readfirstlane(route[RT_IDS + q]);
        const uint8_t *slab = bank.base + (size_t)e * bank.stride;
        const uint8_t *wr = slab + bank.off_dw + (size_t)(r0 + n) * inter + 32u * g;
        const float *srow = (const float *)(slab + bank.off_ds) + (size_t)(r0 >> 7) * nkb;
        if (q != wv) {          /* second slot of this wave (topk > 8) */
#pragma unroll
            for (int u = 0; u < DN_U; u++) {
                const uint32_t c = min((uint32_t)u, nch - 1u);
                pre[u] = ghip_chunk_load(wr + (size_t)c * 128);
                sc[u] = srow[c];
            }
            ghip_wcopy(hs + (size_t)q * inter, h + (size_t)q * inter, inter >> 3, lane);
        }
        const bool exact = bank.nan_flags && bank.nan_flags[e];
        const uint16_t *ha = hs + (size_t)q * inter + 32u * g;
        ghip_f32x4 acc = exact ? down_rows<true>(wr, srow, ha, nch, pre, sc)
                               : down_rows<false>(wr, srow, ha, nch, pre, sc);
        if (g == 0) oq[q][n] = acc[0];
    }
    __syncthreads();
    if (tid < 16) {
        float y = 0.0f;
        for (uint32_t q = 0; q < nsel; q++) {
            float eo = ghip_bf16_round(oq[q][tid]);
            float c = ghip_bf16_round(eo * __uint_as_float(route[RT_W + q]));
            y = ghip_bf16_round(y + c);
        }
        out[r0 + tid] = (uint16_t)ghip_bf16_bits(y);
    }
}

/* ------------------------------------------------------------------------ */

extern "C" hipError_t ghip_launch_moe_decode(const GhipBank *bank,
                                             const uint16_t *x,
                                             const float *logits,
                                             const int32_t *idx, const float *w,
                                             int topk, float limit,
                                             uint16_t *out,
                                             const GhipMoeDecodeWs *ws,
                                             const hipEvent_t *ev,
                                             hipStream_t st) {
    if (!bank || !ws || !x || !out) return hipErrorInvalidValue;
    const uint32_t dim = bank->dim, inter = bank->inter;
    if (topk <= 0 || topk > MD_MAXK || (uint32_t)topk > bank->n_experts)
        return hipErrorInvalidValue;
    if (!logits && (!idx || !w)) return hipErrorInvalidValue;
    if (dim == 0 || inter == 0 || dim % 128 || inter % 128) return hipErrorInvalidValue;
    if (logits && bank->n_experts > RT_MAXE) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) || ((uintptr_t)bank->base & 15) || (bank->stride & 15)
        || (bank->off_gw & 15) || (bank->off_uw & 15) || (bank->off_dw & 15)
        || (bank->off_gs & 3) || (bank->off_us & 3) || (bank->off_ds & 3))
        return hipErrorInvalidValue;
    const size_t lds_gu = (size_t)dim * 2, lds_dn = (size_t)topk * inter * 2;
    if (lds_gu > 64 * 1024 || lds_dn > 64 * 1024) return hipErrorInvalidValue;
    hipEvent_t e0 = ev ? ev[0] : nullptr, e1 = ev ? ev[1] : nullptr;
    hipEvent_t e2 = ev ? ev[2] : nullptr, e3 = ev ? ev[3] : nullptr;
    hipEvent_t e4 = ev ? ev[4] : nullptr, e5 = ev ? ev[5] : nullptr;
    hipError_t e;
    GHIP_LAUNCH(e0, e1, k_moe_route, dim3(1), dim3(64), 0, st, logits, idx, w, topk,
                (int)bank->n_experts, ws->route, ws->err);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GHIP_LAUNCH(e2, e3, k_moe_gateup, dim3((uint32_t)topk * (inter / MD_T)),
                dim3(MD_NW * 64), lds_gu, st, *bank, x, ws->route, limit, ws->h);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GHIP_LAUNCH(e4, e5, k_moe_down, dim3(dim / MD_T), dim3(MD_NW * 64), lds_dn, st,
                *bank, ws->h, ws->route, out);
    return hipGetLastError();
}
