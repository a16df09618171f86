/*
 * k_moe.hip — K3: routed-MoE decode for one token in ONE launch (gfx950).
 *
 * Computes, for the selected experts e (ascending id) with weights w_e,
 *     g = x . Wg_e^T, u = x . Wu_e^T          (FP8-block dequant, bf16 out)
 *     h = bf16(bf16(silu(min(g,L))) * clip(u,-L,L))
 *     o_e = h . Wd_e^T                        (bf16 out)
 *     y = 0; y = bf16(y + bf16(o_e * w_e)) for e ascending; out = y
 * i.e. c/gmoe.h:210-227 (apus_gmoe_expert) and the combine loop of
 * c/gmoe.h:307-320, with the harness routing (stable top-k of f32 logits,
 * softmax over the k selected) optionally computed on the device.
 *
 * Work decomposition (persistent workgroups, dynamic tickets):
 *   tickets [0, n1)      phase 1: (slot q, 16 rows of gate AND up) -> h[q]
 *   tickets [n1, n1+n2)  phase 2: (slot q, 32 rows of down) -> contrib[q]
 * Tickets are dispensed in order, q-major, so a phase-2 tile only waits
 * (bounded spin on done1[q]) for phase-1 tiles that running workgroups
 * already hold and finish without waiting: deadlock-free at any residency.
 * The last workgroup to finish a 32-row group (done2 counter) runs the
 * ordered combine for those rows; the last workgroup to exit resets the
 * ticket/done1/exit counters, so every counter is zero again when the
 * kernel ends (no memset between launches).
 *
 * GEMV inner loop: as k_linear.hip (16 rows per MFMA group, 64-wide k
 * chunks split over the 8 waves, 16-byte code loads, dequant in registers,
 * v_mfma_f32_16x16x32_bf16, fixed-order cross-wave sums in LDS).
 */
#include "ghip_device.h"
#include "ghip_internal.h"

#define MD_NW 8
#define MD_T1 16                 /* gate/up rows per phase-1 tile */
#define MD_T2 32                 /* down rows per phase-2 tile */
#define MD_MAXK 16               /* max routed slots */
#define MD_C_TICKET 0
#define MD_C_EXIT 1
#define MD_C_DONE1 16
#define MD_C_DONE2 64
/* bound on one wait, in wall_clock64() ticks (100 MHz on gfx9: 2 s) */
#define MD_WAIT_TICKS 200000000ull

struct MdArgs {
    GhipBank bank;
    const uint16_t *x;
    const float *logits;
    const int32_t *idx;
    const float *w;
    int topk;
    float limit;
    uint16_t *out;
    GhipMoeDecodeWs ws;
};

__device__ __forceinline__ uint32_t ld_acquire(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

/* One 16-row MFMA group over this wave's k chunks; B codes at
 * wr (row already offset), A = x in LDS. Two matrices may share the loop. */
template <bool EXACT, int NMAT>
__device__ __forceinline__ void md_rows(const uint8_t *const wr[NMAT],
                                        const float *const srow[NMAT],
                                        const uint16_t *xa, uint32_t nch,
                                        uint32_t wv, ghip_f32x4 acc[NMAT]) {
    constexpr int U = 16 / NMAT;
    for (uint32_t c0 = wv; c0 < nch; c0 += MD_NW * U) {
        ghip_u32x4 buf[NMAT][U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            uint32_t c = c0 + u * MD_NW;
#pragma unroll
            for (int j = 0; j < NMAT; j++)
                if (c < nch) buf[j][u] = __builtin_nontemporal_load(
                    (const ghip_u32x4 *)(wr[j] + (size_t)c * 64));
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            uint32_t c = c0 + u * MD_NW;
            if (c < nch) {
                ghip_bf16x8 a0 = *(const ghip_bf16x8 *)(xa + c * 64);
                ghip_bf16x8 a1 = *(const ghip_bf16x8 *)(xa + c * 64 + 8);
#pragma unroll
                for (int j = 0; j < NMAT; j++) {
                    ghip_bf16x8 b0, b1;
                    ghip_deq16<EXACT>(buf[j][u], srow[j][c >> 1], b0, b1);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc[j], 0, 0, 0);
                }
            }
        }
    }
}

/* Routing into LDS: sel_e ascending expert ids, sel_w their weights.
 * Returns the number of distinct selected experts. */
__device__ __forceinline__ int md_route(const MdArgs &a, int32_t *sel_e, float *sel_w,
                        int32_t *tmp_e, float *tmp_w, int *nsel_lds) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const int k = a.topk, E = (int)a.bank.n_experts;
    if (tid < 64) {
        if (a.logits) {
            /* stable top-k: k passes of (max value, lowest index) */
            uint64_t taken[4] = {0, 0, 0, 0};     /* up to 64*4*64 experts */
            for (int j = 0; j < k; j++) {
                float bv = 0.0f;
                int bi = -1;
                int slot = 0;
                for (int i = (int)lane; i < E; i += 64, slot++) {
                    if (slot < 256 && ((taken[slot >> 6] >> (slot & 63)) & 1ull)) continue;
                    float v = a.logits[i];
                    if (bi < 0 || v > bv) { bv = v; bi = i; }
                }
                for (int off = 32; off > 0; off >>= 1) {
                    float ov = __shfl_xor(bv, off, 64);
                    int oi = __shfl_xor(bi, off, 64);
                    bool better = (oi >= 0) && (bi < 0 || ov > bv || (ov == bv && oi < bi));
                    if (better) { bv = ov; bi = oi; }
                }
                if (bi >= 0 && (bi & 63) == (int)lane) {
                    int s = bi >> 6;
                    if (s < 256) taken[s >> 6] |= 1ull << (s & 63);
                }
                if (lane == 0) { tmp_e[j] = bi; tmp_w[j] = bv; }
            }
            if (lane == 0) {
                float m = tmp_w[0], ssum = 0.0f;
                for (int j = 0; j < k; j++) {
                    tmp_w[j] = expf(tmp_w[j] - m);
                    ssum = ssum + tmp_w[j];
                }
                for (int j = 0; j < k; j++) tmp_w[j] = tmp_w[j] / ssum;
            }
        } else if (lane < (uint32_t)k) {
            tmp_e[lane] = a.idx[lane];
            tmp_w[lane] = a.w[lane];
        }
    }
    __syncthreads();
    if (tid == 0) {
        /* ascending expert id; a repeated id keeps its first slot, as the
         * reference's first-match slot lookup (c/gmoe.h:309-312) */
        int n = 0;
        for (int j = 0; j < k; j++) {
            int e = tmp_e[j];
            bool dup = false;
            for (int q = 0; q < j; q++) dup |= (tmp_e[q] == e);
            if (dup) continue;
            if (e < 0 || e >= E) {
                atomicOr(a.ws.err, 2u);
                continue;
            }
            int p = n++;
            while (p > 0 && sel_e[p - 1] > e) {
                sel_e[p] = sel_e[p - 1];
                sel_w[p] = sel_w[p - 1];
                p--;
            }
            sel_e[p] = e;
            sel_w[p] = tmp_w[j];
        }
        *nsel_lds = n;
    }
    __syncthreads();
    /* wave-uniform (scalar) so every loop bound derived from it is uniform */
    return __builtin_amdgcn_readfirstlane(*nsel_lds);
}

__global__ __launch_bounds__(MD_NW * 64) void k_moe_decode(MdArgs a) {
    extern __shared__ __align__(16) uint16_t lds[];   /* x [dim] | h [inter] */
    __shared__ float red[2][MD_NW][16];
    __shared__ int32_t sel_e[MD_MAXK], tmp_e[MD_MAXK];
    __shared__ float sel_w[MD_MAXK], tmp_w[MD_MAXK];
    __shared__ int nsel_lds;
    __shared__ uint32_t tk_lds;
    __shared__ int last_lds;

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t dim = a.bank.dim, inter = a.bank.inter;
    uint16_t *xs = lds;
    uint16_t *hs = lds + dim;
    uint32_t *cnt = a.ws.counters;

    const int nsel = md_route(a, sel_e, sel_w, tmp_e, tmp_w, &nsel_lds);
    for (uint32_t i = tid; i < (dim >> 3); i += MD_NW * 64)
        *(ghip_u32x4 *)(xs + (i << 3)) = *(const ghip_u32x4 *)(a.x + (i << 3));
    __syncthreads();

    const uint32_t tiles1 = inter / MD_T1, tiles2 = dim / MD_T2;
    const uint32_t n1 = (uint32_t)nsel * tiles1, n2 = (uint32_t)nsel * tiles2;
    const uint32_t nkb_g = (dim + 127) >> 7, nkb_d = (inter + 127) >> 7;

    for (;;) {
        /* No per-lane branch may sit in this loop: with `if (tid == 0)` at
         * both the end of the body (completion atomics) and the top (ticket
         * grab), the compiler threads the two across the back edge and lanes
         * 1..63 of wave 0 re-enter the tile body without a fresh ticket — an
         * endless loop. Counter traffic is therefore done by all of wave 0
         * under a wave-uniform branch with lane-0-valued atomics, and every
         * value that steers the loop is made scalar with readfirstlane. */
        if (wv == 0) {
            uint32_t v = atomicAdd(cnt + MD_C_TICKET, lane == 0 ? 1u : 0u);
            tk_lds = __builtin_amdgcn_readfirstlane(v);
        }
        __syncthreads();
        const uint32_t t = __builtin_amdgcn_readfirstlane(tk_lds);
        __syncthreads();
        if (t >= n1 + n2) break;
        if (t < n1) {
            /* ---- phase 1: 16 rows of gate and up for slot q ---- */
            const uint32_t q = t / tiles1, r0 = (t - q * tiles1) * MD_T1;
            const uint8_t *slab = a.bank.base + (size_t)sel_e[q] * a.bank.stride;
            const bool exact = a.bank.nan_flags && a.bank.nan_flags[sel_e[q]];
            const uint8_t *wr[2] = {
                slab + a.bank.off_gw + (size_t)(r0 + n) * dim + 16u * g,
                slab + a.bank.off_uw + (size_t)(r0 + n) * dim + 16u * g };
            const float *sr[2] = {
                (const float *)(slab + a.bank.off_gs) + (size_t)(r0 >> 7) * nkb_g,
                (const float *)(slab + a.bank.off_us) + (size_t)(r0 >> 7) * nkb_g };
            ghip_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            if (exact) md_rows<true, 2>(wr, sr, xs + 16u * g, dim >> 6, wv, acc);
            else md_rows<false, 2>(wr, sr, xs + 16u * g, dim >> 6, wv, acc);
            if (g == 0) { red[0][wv][n] = acc[0][0]; red[1][wv][n] = acc[1][0]; }
            __syncthreads();
            if (tid < 16) {
                float gs = 0.0f, us = 0.0f;
#pragma unroll
                for (int w = 0; w < MD_NW; w++) { gs += red[0][w][tid]; us += red[1][w][tid]; }
                uint32_t h = ghip_swiglu(ghip_bf16_round(gs), ghip_bf16_round(us), a.limit);
                a.ws.h[(size_t)q * inter + r0 + tid] = (uint16_t)h;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __syncthreads();
            if (wv == 0)
                __hip_atomic_fetch_add(cnt + MD_C_DONE1 + q, lane == 0 ? 1u : 0u,
                                       __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            /* ---- phase 2: 32 rows of down for slot q ---- */
            const uint32_t t2 = t - n1;
            const uint32_t q = t2 / tiles2, r0 = (t2 - q * tiles2) * MD_T2;
            if (wv == 0) {
                /* whole wave 0 polls (uniform loop, scalar exit) */
                const uint64_t t0 = wall_clock64();
                while (__builtin_amdgcn_readfirstlane(
                           ld_acquire(cnt + MD_C_DONE1 + q)) < tiles1) {
                    __builtin_amdgcn_s_sleep(2);
                    if (wall_clock64() - t0 > MD_WAIT_TICKS) {
                        atomicOr(a.ws.err, lane == 0 ? 1u : 0u);
                        break;
                    }
                }
            }
            __syncthreads();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            const uint16_t *hq = a.ws.h + (size_t)q * inter;
            for (uint32_t i = tid; i < (inter >> 3); i += MD_NW * 64)
                *(ghip_u32x4 *)(hs + (i << 3)) =
                    __builtin_nontemporal_load((const ghip_u32x4 *)(hq + (i << 3)));
            __syncthreads();
            const uint8_t *slab = a.bank.base + (size_t)sel_e[q] * a.bank.stride;
            const bool exact = a.bank.nan_flags && a.bank.nan_flags[sel_e[q]];
            const float *sd = (const float *)(slab + a.bank.off_ds);
            const uint8_t *wr[2] = {
                slab + a.bank.off_dw + (size_t)(r0 + n) * inter + 16u * g,
                slab + a.bank.off_dw + (size_t)(r0 + 16 + n) * inter + 16u * g };
            const float *sr[2] = { sd + (size_t)(r0 >> 7) * nkb_d,
                                   sd + (size_t)((r0 + 16) >> 7) * nkb_d };
            ghip_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            if (exact) md_rows<true, 2>(wr, sr, hs + 16u * g, inter >> 6, wv, acc);
            else md_rows<false, 2>(wr, sr, hs + 16u * g, inter >> 6, wv, acc);
            if (g == 0) { red[0][wv][n] = acc[0][0]; red[1][wv][n] = acc[1][0]; }
            __syncthreads();
            if (tid < 32) {
                const uint32_t j = tid >> 4, nn = tid & 15u;
                float ys = 0.0f;
#pragma unroll
                for (int w = 0; w < MD_NW; w++) ys += red[j][w][nn];
                float eo = ghip_bf16_round(ys);
                a.ws.contrib[(size_t)q * dim + r0 + tid] =
                    (uint16_t)ghip_bf16_bits(eo * sel_w[q]);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __syncthreads();
            if (wv == 0) {
                uint32_t old = __hip_atomic_fetch_add(cnt + MD_C_DONE2 + r0 / MD_T2,
                                                      lane == 0 ? 1u : 0u,
                                                      __ATOMIC_ACQ_REL,
                                                      __HIP_MEMORY_SCOPE_AGENT);
                last_lds = __builtin_amdgcn_readfirstlane(old) == (uint32_t)nsel - 1u;
            }
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(last_lds)) {
                /* ordered combine (ascending expert id, bf16 per add) */
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                if (tid < MD_T2) {
                    float y = 0.0f;
                    for (int qq = 0; qq < nsel; qq++) {
                        uint16_t c = __builtin_nontemporal_load(
                            a.ws.contrib + (size_t)qq * dim + r0 + tid);
                        y = ghip_bf16_round(y + ghip_bf16_f32(c));
                    }
                    a.out[r0 + tid] = (uint16_t)ghip_bf16_bits(y);
                }
                if (wv == 0)
                    __hip_atomic_store(cnt + MD_C_DONE2 + r0 / MD_T2, 0u,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    /* last workgroup out resets the shared counters for the next launch */
    if (wv == 0) {
        uint32_t old = __builtin_amdgcn_readfirstlane(__hip_atomic_fetch_add(
            cnt + MD_C_EXIT, lane == 0 ? 1u : 0u, __ATOMIC_ACQ_REL,
            __HIP_MEMORY_SCOPE_AGENT));
        if (old == gridDim.x - 1u) {
            __hip_atomic_store(cnt + MD_C_TICKET, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int q = 0; q < MD_MAXK; q++)
                __hip_atomic_store(cnt + MD_C_DONE1 + q, 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(cnt + MD_C_EXIT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

extern "C" hipError_t ghip_launch_moe_decode(const GhipBank *bank,
                                             const uint16_t *x,
                                             const float *logits,
                                             const int32_t *idx, const float *w,
                                             int topk, float limit,
                                             uint16_t *out,
                                             const GhipMoeDecodeWs *ws,
                                             hipStream_t st) {
    if (!bank || !ws || !x || !out) return hipErrorInvalidValue;
    const uint32_t dim = bank->dim, inter = bank->inter;
    if (topk <= 0 || topk > MD_MAXK || (uint32_t)topk > bank->n_experts)
        return hipErrorInvalidValue;
    if (logits && bank->n_experts > 64u * 256u) return hipErrorInvalidValue;
    if (dim == 0 || inter == 0 || dim % 64 || inter % 64 || dim % MD_T2)
        return hipErrorInvalidValue;
    if (MD_C_DONE2 + dim / MD_T2 > GHIP_MOE_DEC_COUNTERS) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) || ((uintptr_t)bank->base & 15) || (bank->stride & 15)
        || (bank->off_gw & 15) || (bank->off_uw & 15) || (bank->off_dw & 15)
        || (bank->off_gs & 3) || (bank->off_us & 3) || (bank->off_ds & 3))
        return hipErrorInvalidValue;
    size_t lds = (size_t)(dim + inter) * 2;
    if (lds > 48 * 1024) return hipErrorInvalidValue;
    static int grid = 0;
    if (grid == 0) {
        int dev = 0, ncu = 0, per = 0;
        if (hipGetDevice(&dev) != hipSuccess
            || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess
            || hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_moe_decode,
                                                            MD_NW * 64, lds) != hipSuccess
            || ncu <= 0 || per <= 0)
            grid = 256;
        else
            grid = ncu * per;
    }
    MdArgs a;
    a.bank = *bank;
    a.x = x;
    a.logits = logits;
    a.idx = idx;
    a.w = w;
    a.topk = topk;
    a.limit = limit;
    a.out = out;
    a.ws = *ws;
    hipLaunchKernelGGL(k_moe_decode, dim3((uint32_t)grid), dim3(MD_NW * 64), lds,
                       st, a);
    return hipGetLastError();
}
