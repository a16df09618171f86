/*
 * k_moe.hip — K3: routed-MoE decode for one token (gfx950), and the router.
 *
 * The decode is ONE persistent launch (one workgroup per CU, all resident
 * at once) with three phases:
 *   route    one wave per workgroup (every workgroup routes redundantly, so
 *            none waits for another): the harness routing (stable top-k of
 *            f32 logits, ties -> lower id) or given idx/w, a repeated id
 *            keeping its first slot (c/gmoe.h:309-312). Only the selected
 *            ids are needed to start streaming; the softmax weights (kept
 *            at their ascending-id combine positions) are computed later.
 *   gate/up  per (slot q, 16 rows) the g and u GEMVs over dim with the FP8
 *            dequant fused (bit-exact weights) and the SwiGLU epilogue of
 *            c/gmoe.h:217-225 -> h[q] in HBM.
 *   down     per 16 output rows: wave q computes slot q's down GEMV
 *            (h[q] . Wd^T over all of inter), then the ascending-expert
 *            combine y = bf16(y + bf16(bf16(o)*w)) (c/gmoe.h:307-320) runs
 *            in-workgroup -- no float atomics, no cross-workgroup reduction,
 *            deterministic.
 * Hand-off of h between the phases: two h values per 32-bit word, stored
 * with a device-coherent store into a buffer that holds only the sentinel
 * MD_HSENT until this launch writes it (two buffers alternate between
 * launches; each launch refills the other one, which the launch before it
 * read and the launch after it writes); a reader polls the words with
 * device-coherent loads until none is the sentinel (bounded). No fence,
 * counter or barrier between workgroups is involved, and a reader needs
 * nothing but the words it reads.
 *
 * Weight streaming: waves pull their 16-row chunks (128-wide k, one scale
 * block) through registers (whole-line 16-byte loads), write each to a
 * wave-private LDS slot and read it back in the MFMA layout; each down wave
 * loads its first chunks, then awaits its own slot's h (no workgroup
 * barrier) and streams its rows as soon as it is in. The GEMV inner step
 * dequantizes in registers and reduces over k on MFMA with the activation
 * (x or h) from LDS as the A operand.
 */
#include "ghip_device.h"
#include <type_traits>
#include "ghip_internal.h"

#define MD_NW 8                  /* waves per workgroup */
#define MD_T 16                  /* rows per tile (one MFMA group) */
#define MD_MAXK 16               /* max routed slots */
#define MD_LDS_MAX (144 * 1024)  /* dynamic LDS limit of the decode kernel */
#define MD_SPIN_MAX (1u << 18)   /* bounded wait for the device-wide hand-off */
#define MD_HSENT 0xffffffffu     /* an h word not written yet in this launch */

/* Two h values (bf16 bits, lo = the even row) as one hand-off word. The
 * sentinel would be a pair of all-ones NaNs (a NaN whose 32-bit source has
 * every mantissa bit set, as the bf16 narrowing keeps NaN payloads): that
 * pair is stored with the even row's NaN payload one lower (0xfffe), still
 * a NaN of the same sign, so every word a launch stores differs from the
 * sentinel. */
__device__ __forceinline__ uint32_t md_hpack(uint32_t lo, uint32_t hi) {
    const uint32_t wd = lo | (hi << 16);
    return wd == MD_HSENT ? wd - 1u : wd;
}

/* ------------------------------------------------------------------------ */
/* routing                                                                  */
/* ------------------------------------------------------------------------ */

#define RT_MAXE 512              /* experts a routing wave can hold (8 per lane) */

/* Monotone u32 key of a float: a larger value gives a larger key, and -0
 * and +0 share one (they compare equal in the reference). Keys are >= 1, so
 * 0 marks an empty or already-taken slot. */
__device__ __forceinline__ uint32_t rt_key(float v) {
    uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return u ? u : 1u;
}

/* the value of a key (the inverse of rt_key for every non-NaN value) */
__device__ __forceinline__ float rt_val(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

/* k = max of k and k moved by a DPP pattern; lanes without a source keep
 * k (the moved value is 0 there, the identity of an unsigned max, so the
 * move folds into one v_max_u32_dpp) */
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t rt_dpp(uint32_t k) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, CTRL, ROWMASK, 0xf, true);
    return o > k ? o : k;
}

/* Wave max on DPP (VALU lane moves, no LDS round trips): row shifts leave
 * each row's result in its lane 15, two row broadcasts carry it to lane
 * 63, read back as a wave-uniform value. */
__device__ __forceinline__ uint32_t rt_wave_max(uint32_t k) {
    k = rt_dpp<0x111, 0xf>(k);           /* row_shr:1 */
    k = rt_dpp<0x112, 0xf>(k);           /* row_shr:2 */
    k = rt_dpp<0x114, 0xf>(k);           /* row_shr:4 */
    k = rt_dpp<0x118, 0xf>(k);           /* row_shr:8 */
    k = rt_dpp<0x142, 0xa>(k);           /* row_bcast:15 */
    k = rt_dpp<0x143, 0xc>(k);           /* row_bcast:31 */
    return (uint32_t)__builtin_amdgcn_readlane((int)k, 63);
}

/* Stable top-k by one wave (c/gmoe.h:175-189: larger first, ties to the
 * lower index): slot s of lane l holds the key of index R l + s (0 =
 * empty), so each lane holds a run of consecutive indices and a lower lane
 * lower ones. Each lane first sorts its R keys in descending order (a
 * bubble network that swaps only on a strictly larger key, so equal keys
 * keep the lower index first). Each of the k rounds then takes one 32-bit
 * DPP wave max of the lanes' heads; of the lanes whose head equals it the
 * lowest one holds the lowest index with that key (its head is its lowest
 * such index, and lower lanes hold lower indices), and it drops its head.
 * Lane j < k returns pick j's index and its key in mykey. KC > 0: the
 * count is KC at compile time (topk == KC), so the rounds unroll and one
 * round's remaining register moves overlap the next round's wave max. */
template <int R, int KC = 0>
__device__ __forceinline__ int rt_select_n(uint32_t (&key)[R], int topk, uint32_t &mykey) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t ss[R];
#pragma unroll
    for (int s = 0; s < R; s++) ss[s] = (uint32_t)s;
#pragma unroll
    for (int i = 0; i < R - 1; i++)
#pragma unroll
        for (int j = 0; j < R - 1 - i; j++) {
            const bool sw = key[j + 1] > key[j];
            const uint32_t ka = key[j], kb = key[j + 1], sa = ss[j], sb = ss[j + 1];
            key[j] = sw ? kb : ka;
            key[j + 1] = sw ? ka : kb;
            ss[j] = sw ? sb : sa;
            ss[j + 1] = sw ? sa : sb;
        }
    int myid = -1;
    mykey = 0u;
    const int nk = KC > 0 ? KC : topk;
#pragma unroll
    for (int j = 0; j < nk; j++) {
        const uint32_t wm = rt_wave_max(key[0]);
        const uint32_t wl = (uint32_t)__builtin_ctzll(__ballot(key[0] == wm));
        const uint32_t widx = wl * (uint32_t)R + (uint32_t)__builtin_amdgcn_readlane((int)ss[0], wl);
        if (lane == wl) {
#pragma unroll
            for (int s = 0; s + 1 < R; s++) {
                key[s] = key[s + 1];
                ss[s] = ss[s + 1];
            }
            key[R - 1] = 0u;
        }
        if ((int)lane == j) {
            myid = (int)widx;
            mykey = wm;
        }
    }
    return myid;
}

/* rt_select_n with the model's top-8 unrolled */
template <int R>
__device__ __forceinline__ int rt_select(uint32_t (&key)[R], int topk, uint32_t &mykey) {
    return topk == 8 ? rt_select_n<R, 8>(key, 8, mykey) : rt_select_n<R>(key, topk, mykey);
}

/* Selection of the harness routing from logits by one wave: the stable
 * top-k (ties -> lower id). Lane j < topk returns pick j's id and its logit
 * (selection order). R logits per lane. */
template <int R>
__device__ __forceinline__ int md_select(const float *__restrict__ logits, int topk, int E,
                                         float &mylog) {
    const int lane = threadIdx.x & 63;
    /* all R loads are issued before any is used: the index is clamped
     * rather than the load predicated, which would wait for each load
     * inside its own branch (R serial memory round trips) */
    float v[R];
#pragma unroll
    for (int s = 0; s < R; s++) {
        const int i = lane * R + s;
        v[s] = logits[i < E ? i : E - 1];
    }
    /* an unconditional use pins each load here (the compiler would
     * otherwise sink a load into the branch that consumes it) */
#pragma unroll
    for (int s = 0; s < R; s++) asm volatile("" ::"v"(v[s]));
    uint32_t key[R];
#pragma unroll
    for (int s = 0; s < R; s++) key[s] = lane * R + s < E ? rt_key(v[s]) : 0u;
    uint32_t mk;
    const int myid = rt_select<R>(key, topk, mk);
    mylog = rt_val(mk);
    return myid;
}

#define GU_NW 8                  /* waves per workgroup (two per SIMD) */
#define GU_IPW 4                 /* items per workgroup pass (2 waves each) */
#define GU_R 2                   /* LDS slots per wave (gate + up chunk each) */
#define GU_STG 4096              /* bytes per stage */
#define DN_R 3                   /* down LDS slots per wave (one chunk each) */
#define DN_STG 2048

/* Per-workgroup shared state (static LDS). Slots: the kept routing picks
 * in selection order (logits) or given order (idx); sel[q] is slot q's
 * expert. Combine positions: position i is the i-th smallest kept expert
 * id; wt[i] is its weight and oq[i] its output rows. */
struct MdShared {
    int32_t sel[MD_MAXK];
    float wt[MD_MAXK];
    float lg[MD_MAXK];           /* logits path: slot q's logit */
    int32_t te[MD_MAXK];
    float tw[MD_MAXK];
    uint32_t nsel;
    float red[GU_IPW][2][2][16];
    float oq[MD_MAXK][16];
    float sred[MD_NW][16];       /* shared expert: gate/up partials per wave */
    float sdown[MD_NW][16];      /* shared expert: down partials per wave */
};

#define MD_SH_SLOT MD_MAXK       /* the shared expert's h words: slot 16 */
#define SH_GRP 5                 /* shared gate/up chunks in flight per wave (x: <= 128
                                    vectors, two per lane) */
#define SD_GRP 4                 /* shared down chunks in flight per wave */

/* Phase A, wave 0 only: the routing picks into sh.sel / sh.nsel. Given
 * idx/w: a repeated id keeps its first slot (c/gmoe.h:309-312), invalid ids
 * are dropped and flagged; kept slots stay in the given order, their
 * weights at their ascending-id combine positions. Logits: the selected ids
 * and their logits (the weights come later, md_route_finish). */
__device__ __forceinline__ void md_route_ids(const float *__restrict__ logits,
                                             const int32_t *__restrict__ idx,
                                             const float *__restrict__ w, int topk, int E,
                                             MdShared &sh, uint32_t *__restrict__ err) {
    const int lane = threadIdx.x & 63;
    if (logits) {
        float mylog;
        const int myid = E <= 5 * 64 ? md_select<5>(logits, topk, E, mylog)
                                     : md_select<8>(logits, topk, E, mylog);
        if (lane < topk) {
            sh.sel[lane] = myid;
            sh.lg[lane] = mylog;
        }
        if (lane == 0) sh.nsel = (uint32_t)topk;
        return;
    }
    /* given routing: the loads of all slots first (one round trip) */
    const int e = lane < topk ? idx[lane] : -1;
    const float wj = lane < topk ? w[lane] : 0.0f;
    bool keep = lane < topk;
    if (keep && (e < 0 || e >= E)) {
        keep = false;
        if (err) atomicOr(err, 2u);
    }
    /* slot q is uniform: read it with readlane, not a lane permute */
    for (int q = 0; q < topk; q++)
        if (q < lane && __builtin_amdgcn_readlane(e, q) == e) keep = false;
    const uint64_t kept = __ballot(keep);
    const int slot = (int)__popcll(kept & ((1ull << lane) - 1ull));
    int rank = 0;
    for (int q = 0; q < topk; q++)
        rank += ((kept >> q) & 1u) && __builtin_amdgcn_readlane(e, q) < e;
    if (keep) {
        sh.sel[slot] = e;
        sh.wt[rank] = wj;
    }
    if (lane == 0) sh.nsel = (uint32_t)__popcll(kept);
}

/* Logits path, wave 0, after phase A: softmax over the k selected logits in
 * slot order (m = slot 0's logit, e_q = expf(l_q - m), s = e_0 + e_1 + ...
 * ascending q, w = e / s), each weight stored at its slot's combine
 * position (ascending id). */
__device__ __forceinline__ void md_route_finish(MdShared &sh, int topk) {
    const int lane = threadIdx.x & 63;
    const int myid = lane < topk ? sh.sel[lane] : 0x7fffffff;
    const float mylog = lane < topk ? sh.lg[lane] : 0.0f;
    const float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                  __builtin_bit_cast(int, mylog), 0));
    const float ej = expf(mylog - m);
    float ssum = 0.0f;
    for (int j = 0; j < topk; j++)
        ssum = ssum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                     __builtin_bit_cast(int, ej), j));
    int rank = 0;
    for (int j = 0; j < topk; j++) rank += __builtin_amdgcn_readlane(myid, j) < myid;
    if (lane < topk) sh.wt[rank] = ej / ssum;
}

/* Phase B: items = (slot q, 16 rows): gate and up GEMVs over dim and the
 * SwiGLU; workgroup b takes item groups b, b + G, ... of GU_IPW items; wave
 * w streams item (w / 2)'s half (w % 2) of K through registers and a
 * wave-private pair of LDS slots (no barriers inside the stream); the
 * halves are summed in LDS in a fixed order (deterministic). The 16 h
 * values of an item go to hw[q] in HBM as 8 hand-off words (lanes 0..7 of
 * the item's even wave, two rows each). */
__device__ __forceinline__ void md_phase_gateup(const GhipBank &bank, const uint16_t *xs,
                                                uint8_t *ring_base, MdShared &sh,
                                                float limit, uint32_t *hw) {
    const uint32_t dim = bank.dim, inter = bank.inter;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nsel = __builtin_amdgcn_readfirstlane(sh.nsel);
    const uint32_t tiles = inter / MD_T, items = nsel * tiles;
    const uint32_t groups = (items + GU_IPW - 1) / GU_IPW;
    uint8_t *ring = ring_base + wv * (GU_R * GU_STG);
    const uint32_t nch = dim >> 7, nkb = dim >> 7;
    const uint32_t half = wv & 1u, slot = wv >> 1;
    const uint32_t c0 = half ? nch / 2 : 0u, c1 = half ? nch : nch / 2;
    const uint32_t nc = c1 - c0;
    const ghip_cdma d = ghip_cdma_offsets(lane, dim);
    const uint32_t n = lane & 15u, g = lane >> 4;

    for (uint32_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {
        const uint32_t it = grp * GU_IPW + slot;
        const bool live = it < items;
        uint32_t q = 0, r0 = 0;
        if (live) {
            q = it / tiles;
            r0 = (it - q * tiles) * MD_T;
            const uint32_t e = (uint32_t)__builtin_amdgcn_readfirstlane(sh.sel[q]);
            const uint8_t *slab = bank.base + (size_t)e * bank.stride;
            const uint8_t *wg = slab + bank.off_gw + (size_t)r0 * dim;
            const uint8_t *wu = slab + bank.off_uw + (size_t)r0 * dim;
            const float *sg = (const float *)(slab + bank.off_gs) + (size_t)(r0 >> 7) * nkb;
            const float *su = (const float *)(slab + bank.off_us) + (size_t)(r0 >> 7) * nkb;
            /* stage t (gate chunk + up chunk) through registers: written to
             * LDS slot t % 2, then the registers take stage t + 1 while
             * stage t is computed (one stage in flight per wave: deeper
             * made the step slower, as with the LDS-DMA ring) */
            ghip_u32x4 ga0, ga1, ua0, ua1;
            auto ld = [&](uint32_t t, ghip_u32x4 &g0, ghip_u32x4 &g1, ghip_u32x4 &u0,
                          ghip_u32x4 &u1) {
                ghip_rl_load(wg, d, c0 + t, g0, g1);
                ghip_rl_load(wu, d, c0 + t, u0, u1);
            };
            ld(0u, ga0, ga1, ua0, ua1);
            /* the expert's NaN-code flag and the first chunk's scales are
             * read after the first stage is on its way, so their round
             * trips (the scales' line is cold) overlap the stage's instead
             * of following it */
            __builtin_amdgcn_sched_barrier(0);
            const bool exact = ghip_sload_u32(bank.nan_flags, e) != 0u;
            const float scg0 = ghip_sload(sg, c0), scu0 = ghip_sload(su, c0);
            __builtin_amdgcn_sched_barrier(0);
            ghip_f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
            for (uint32_t t = 0; t < nc; t++) {
                uint8_t *buf = ring + (t & 1u) * GU_STG;
                ghip_rl_store(buf, lane, ga0, ga1);
                ghip_rl_store(buf + 2048, lane, ua0, ua1);
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1u < nc) ld(t + 1u, ga0, ga1, ua0, ua1);
                __builtin_amdgcn_sched_barrier(0);
                const uint32_t c = c0 + t;
                /* codes, activations and scales requested before any is
                 * used: one LDS wait covers them */
                const ghip_chunk cg = ghip_cdma_read(buf, n, g);
                const ghip_chunk cu = ghip_cdma_read(buf + 2048, n, g);
                ghip_bf16x8 xa[4];
                ghip_read_a4(xs + c * 128u + 32u * g, xa);
                const float scg = t ? ghip_sload(sg, c) : scg0;
                const float scu = t ? ghip_sload(su, c) : scu0;
                __builtin_amdgcn_sched_barrier(0);
                if (exact) {
                    ghip_chunk_mfma_a<true>(cg, scg, xa, ag);
                    ghip_chunk_mfma_a<true>(cu, scu, xa, au);
                } else {
                    ghip_chunk_mfma_a<false>(cg, scg, xa, ag);
                    ghip_chunk_mfma_a<false>(cu, scu, xa, au);
                }
            }
            if (g == 0) {
                sh.red[slot][half][0][n] = ag[0];
                sh.red[slot][half][1][n] = au[0];
            }
        }
        __syncthreads();
        if (live && half == 0 && lane < 8) {      /* fixed order: half 0 + half 1 */
            uint32_t hv[2];
#pragma unroll
            for (uint32_t k = 0; k < 2; k++) {
                const uint32_t r = 2u * lane + k;
                const float gs = sh.red[slot][0][0][r] + sh.red[slot][1][0][r];
                const float us = sh.red[slot][0][1][r] + sh.red[slot][1][1][r];
                hv[k] = ghip_swiglu(ghip_bf16_round(gs), ghip_bf16_round(us), limit);
            }
            /* rows 2j and 2j + 1 in one word, stored device-coherently: a
             * word that is not the sentinel is this launch's, on any XCD */
            __hip_atomic_store(hw + (size_t)q * (inter / 2u) + r0 / 2u + lane,
                               md_hpack(hv[0], hv[1]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
}

/* The shared expert's gate/up rows 8hb .. 8hb + 7 (c/gmoe.h:325-336: every
 * token runs it, so it needs no routing and waves 1..7 stream it while
 * wave 0 routes). One 16-row chunk holds the gate rows (chunk rows 0..7)
 * and the up rows (chunk rows 8..15) of one 128-wide k block, each half
 * dequantized with its own matrix's block scale, so one MFMA chunk gives
 * both. Wave w = 1..7 takes k blocks [(w-1) nch / 7, w nch / 7), all of
 * them requested before the first is used (SH_GRP at a time), with its x
 * slices staged in its own LDS area, and leaves its fp32 partial sums in
 * sh.sred[w] (summed in a fixed order after the routing barrier).
 * wbuf: the wave's 8 KB area (two 2 KB chunk slots, then the x slices). */
template <bool EXACT>
__device__ __forceinline__ void md_shared_gu_blocks(const uint8_t *gw, const uint8_t *uw,
                                                    const float *sg, const float *su,
                                                    const uint16_t *__restrict__ x,
                                                    const ghip_cdma &d, uint32_t c0,
                                                    uint32_t c1, uint8_t *wbuf,
                                                    ghip_f32x4 &acc) {
    const uint32_t lane = threadIdx.x & 63u, n = lane & 15u, g = lane >> 4;
    uint16_t *xw = (uint16_t *)(wbuf + 4096u);
    for (uint32_t cb = c0; cb < c1; cb += SH_GRP) {
        const uint32_t cn = min(c1 - cb, (uint32_t)SH_GRP);
        /* the x slice first (its wait then covers it alone), then the
         * chunks: cn * 16 <= 80 vectors of 16 bytes, two per lane (index
         * clamped, a duplicate rewrites the last vector with its own value) */
        const uint32_t xv_i = min(lane, cn * 16u - 1u), xv_j = min(lane + 64u, cn * 16u - 1u);
        const ghip_u32x4 xv = *(const ghip_u32x4 *)(x + (size_t)cb * 128u + 8u * xv_i);
        const ghip_u32x4 xw2 = *(const ghip_u32x4 *)(x + (size_t)cb * 128u + 8u * xv_j);
        ghip_u32x4 a0[SH_GRP], a1[SH_GRP];
#pragma unroll
        for (uint32_t j = 0; j < SH_GRP; j++) {
            const uint32_t cj = cb + min(j, cn - 1u);
            const uint8_t *pg = gw + (size_t)cj * 128u, *pu = uw + (size_t)cj * 128u;
            a0[j] = __builtin_nontemporal_load((const ghip_u32x4 *)(pg + d.off0));
            a1[j] = __builtin_nontemporal_load((const ghip_u32x4 *)(pu + d.off1));
        }
        ((ghip_u32x4 *)xw)[xv_i] = xv;
        ((ghip_u32x4 *)xw)[xv_j] = xw2;
#pragma unroll
        for (uint32_t j = 0; j < SH_GRP; j++) {
            if (j < cn) {
                uint8_t *buf = wbuf + (j & 1u) * 2048u;
                ghip_rl_store(buf, lane, a0[j], a1[j]);
                const ghip_chunk ck = ghip_cdma_read(buf, n, g);
                ghip_bf16x8 xa[4];
                ghip_read_a4(xw + j * 128u + 32u * g, xa);
                const float scg = ghip_sload(sg, cb + j), scu = ghip_sload(su, cb + j);
                ghip_chunk_mfma_a<EXACT>(ck, n < 8u ? scg : scu, xa, acc);
            }
        }
    }
}

__device__ __forceinline__ void md_shared_gateup(const GhipBank &bank,
                                                 const uint16_t *__restrict__ x,
                                                 uint8_t *wbuf, uint32_t hb, MdShared &sh) {
    const uint32_t dim = bank.dim, lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nch = dim >> 7, nkb = dim >> 7;
    const uint32_t c0 = (wv - 1u) * nch / (MD_NW - 1u), c1 = wv * nch / (MD_NW - 1u);
    const uint32_t E = bank.n_experts, r0 = hb * 8u;
    const uint8_t *slab = bank.base + (size_t)E * bank.stride;
    /* gate rows r0.. at chunk rows 0..7; up rows r0.. at chunk rows 8..15,
     * whose offsets (ghip_cdma_offsets) count from chunk row 0: the up base
     * is taken 8 rows back */
    const uint8_t *gw = slab + bank.off_gw + (size_t)r0 * dim;
    const uint8_t *uw = slab + bank.off_uw + (size_t)r0 * dim - (size_t)8u * dim;
    const float *sg = (const float *)(slab + bank.off_gs) + (size_t)(r0 >> 7) * nkb;
    const float *su = (const float *)(slab + bank.off_us) + (size_t)(r0 >> 7) * nkb;
    const ghip_cdma d = ghip_cdma_offsets(lane, dim);
    ghip_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (ghip_sload_u32(bank.nan_flags, E) != 0u)
        md_shared_gu_blocks<true>(gw, uw, sg, su, x, d, c0, c1, wbuf, acc);
    else
        md_shared_gu_blocks<false>(gw, uw, sg, su, x, d, c0, c1, wbuf, acc);
    if ((lane >> 4) == 0) sh.sred[wv][lane] = acc[0];
}

/* After the routing barrier: the shared expert's 8 h values of rows 8hb..
 * (lane j < 4 of the calling wave: rows 8hb + 2j and 8hb + 2j + 1): the
 * partial sums of waves 1..7 in that order, the reference's bf16 roundings
 * and SwiGLU, stored as hand-off words (as the routed slots' h) in slot
 * MD_SH_SLOT. */
__device__ __forceinline__ void md_shared_h(const MdShared &sh, uint32_t hb, uint32_t inter,
                                            float limit, uint32_t *hw) {
    const uint32_t lane = threadIdx.x & 63u;
    if (lane < 4u) {
        uint32_t hv[2];
#pragma unroll
        for (uint32_t k = 0; k < 2; k++) {
            const uint32_t r = 2u * lane + k;
            float gs = sh.sred[1][r], us = sh.sred[1][8u + r];
#pragma unroll
            for (uint32_t w = 2; w < MD_NW; w++) {
                gs = gs + sh.sred[w][r];
                us = us + sh.sred[w][8u + r];
            }
            hv[k] = ghip_swiglu(ghip_bf16_round(gs), ghip_bf16_round(us), limit);
        }
        __hip_atomic_store(hw + (size_t)MD_SH_SLOT * (inter / 2u) + hb * 4u + lane,
                           md_hpack(hv[0], hv[1]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

/* The shared expert's down rows r0 .. r0 + 15 over the calling wave's
 * share of inter, k blocks [wv nchd / 8, (wv + 1) nchd / 8), with that
 * share of its h already staged at hss; the fp32 partials go to
 * sh.sdown[wv] (summed in wave order by the combine). Uses the wave's first
 * two down LDS slots before its routed rows do. */
template <bool EXACT>
__device__ __forceinline__ void md_shared_down_blocks(const uint8_t *rows, const float *srow,
                                                      const uint16_t *hss,
                                                      const ghip_cdma &d, uint32_t c0,
                                                      uint32_t c1, uint8_t *ring,
                                                      ghip_f32x4 &acc) {
    const uint32_t lane = threadIdx.x & 63u, n = lane & 15u, g = lane >> 4;
    for (uint32_t cb = c0; cb < c1; cb += SD_GRP) {
        const uint32_t cn = min(c1 - cb, (uint32_t)SD_GRP);
        ghip_u32x4 a0[SD_GRP], a1[SD_GRP];
#pragma unroll
        for (uint32_t j = 0; j < SD_GRP; j++)
            ghip_rl_load(rows, d, cb + min(j, cn - 1u), a0[j], a1[j]);
#pragma unroll
        for (uint32_t j = 0; j < SD_GRP; j++) {
            if (j < cn) {
                uint8_t *buf = ring + (j & 1u) * DN_STG;
                ghip_rl_store(buf, lane, a0[j], a1[j]);
                const ghip_chunk ck = ghip_cdma_read(buf, n, g);
                ghip_bf16x8 ha[4];
                ghip_read_a4(hss + (cb - c0 + j) * 128u + 32u * g, ha);
                ghip_chunk_mfma_a<EXACT>(ck, ghip_sload(srow, cb + j), ha, acc);
            }
        }
    }
}

/* Phase C, down + ordered combine for the 16 output rows at r0: wave q
 * streams slot base + q's 16 rows of Wd over inter through registers and
 * its DN_R LDS slots with h of that slot (in LDS at hs + q * inter) as the
 * A operand and leaves the expert output in sh.oq; md_combine then runs the
 * ordered combine in-workgroup. md_down_prologue loads the first DN_R
 * chunks (so they stream while the wave waits for h). */
/* what md_down_prologue loaded for md_phase_down: the first DN_R chunks,
 * and the expert's NaN-code flag and the first chunk's scale as vector
 * loads issued before the wait for h, so their cold round trips overlap it
 * (the h polling waits for them with its own loads; scalar loads would be
 * waited at once, their SGPRs being spilled to VGPR lanes) */
struct MdDownHead {
    uint32_t flag;
    uint32_t sc0;
    ghip_u32x4 a0, a1, b0, b1, c0, c1;    /* the first three chunks (registers) */
};

__device__ __forceinline__ MdDownHead md_down_prologue(const GhipBank &bank, const MdShared &sh,
                                                       uint32_t r0, uint32_t base) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nsel = __builtin_amdgcn_readfirstlane(sh.nsel);
    MdDownHead hd{};
    if (base + wv >= nsel) return hd;
    const uint32_t inter = bank.inter, nch = inter >> 7, nkb = inter >> 7;
    const uint32_t e = (uint32_t)__builtin_amdgcn_readfirstlane(sh.sel[base + wv]);
    const uint8_t *slab = bank.base + (size_t)e * bank.stride;
    const uint8_t *rows = slab + bank.off_dw + (size_t)r0 * inter;
    const ghip_cdma d = ghip_cdma_offsets(lane, inter);
    ghip_rl_load(rows, d, 0u, hd.a0, hd.a1);
    __builtin_amdgcn_sched_barrier(0);
    ghip_rl_load(rows, d, nch > 1u ? 1u : 0u, hd.b0, hd.b1);
    __builtin_amdgcn_sched_barrier(0);
    ghip_rl_load(rows, d, nch > 2u ? 2u : 0u, hd.c0, hd.c1);
    __builtin_amdgcn_sched_barrier(0);
    const float *srow = (const float *)(slab + bank.off_ds) + (size_t)(r0 >> 7) * nkb;
    hd.flag = __hip_atomic_load(bank.nan_flags + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    hd.sc0 = __hip_atomic_load((const uint32_t *)srow, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
    return hd;
}

__device__ __forceinline__ void md_phase_down(const GhipBank &bank, MdShared &sh,
                                              uint32_t r0, uint32_t base, const uint16_t *hs,
                                              uint8_t *ring_base, MdDownHead &hd) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t inter = bank.inter, nch = inter >> 7, nkb = inter >> 7;
    const uint32_t nsel = __builtin_amdgcn_readfirstlane(sh.nsel);
    if (base + wv < nsel) {
        const uint32_t e = (uint32_t)__builtin_amdgcn_readfirstlane(sh.sel[base + wv]);
        /* the slot's combine position: how many kept ids are smaller (the
         * kept ids are distinct) */
        const int32_t si = lane < nsel ? sh.sel[lane] : 0x7fffffff;
        const uint32_t pos = (uint32_t)__popcll(__ballot(si < (int32_t)e));
        const uint8_t *slab = bank.base + (size_t)e * bank.stride;
        const uint8_t *rows = slab + bank.off_dw + (size_t)r0 * inter;
        const float *srow = (const float *)(slab + bank.off_ds) + (size_t)(r0 >> 7) * nkb;
        const bool exact = __builtin_amdgcn_readfirstlane(hd.flag) != 0u;
        const float sc0 = __uint_as_float(__builtin_amdgcn_readfirstlane(hd.sc0));
        const ghip_cdma d = ghip_cdma_offsets(lane, inter);
        uint8_t *ring = ring_base + wv * (DN_R * DN_STG);
        ghip_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        /* chunk t: registers (set t % 3, the first three loaded by the
         * prologue) into LDS slot t % 3, refilled with chunk t + 3 (three
         * chunks in flight: the down rows stream after the hand-off, where
         * deeper helps) */
        auto step = [&](auto refill_c, uint32_t t, uint32_t j, ghip_u32x4 &v0, ghip_u32x4 &v1) {
            uint8_t *buf = ring + j * DN_STG;
            ghip_rl_store(buf, lane, v0, v1);
            if constexpr (decltype(refill_c)::value) {
                __builtin_amdgcn_sched_barrier(0);
                ghip_rl_load(rows, d, t + 3u, v0, v1);
                __builtin_amdgcn_sched_barrier(0);
            }
            const ghip_chunk cw = ghip_cdma_read(buf, n, g);
            ghip_bf16x8 ha[4];
            ghip_read_a4(hs + (size_t)wv * inter + t * 128u + 32u * g, ha);
            const float sc = t ? ghip_sload(srow, t) : sc0;
            __builtin_amdgcn_sched_barrier(0);
            if (exact) ghip_chunk_mfma_a<true>(cw, sc, ha, acc);
            else ghip_chunk_mfma_a<false>(cw, sc, ha, acc);
        };
        using RF = std::true_type;
        using NR = std::false_type;
        uint32_t t = 0;
        for (; t + 5u < nch; t += 3) {
            step(RF{}, t, 0u, hd.a0, hd.a1);
            step(RF{}, t + 1u, 1u, hd.b0, hd.b1);
            step(RF{}, t + 2u, 2u, hd.c0, hd.c1);
        }
        const uint32_t rem = nch - t;
        if (rem == 5u) {
            step(RF{}, t, 0u, hd.a0, hd.a1);
            step(RF{}, t + 1u, 1u, hd.b0, hd.b1);
            step(NR{}, t + 2u, 2u, hd.c0, hd.c1);
            step(NR{}, t + 3u, 0u, hd.a0, hd.a1);
            step(NR{}, t + 4u, 1u, hd.b0, hd.b1);
        } else if (rem == 4u) {
            step(RF{}, t, 0u, hd.a0, hd.a1);
            step(NR{}, t + 1u, 1u, hd.b0, hd.b1);
            step(NR{}, t + 2u, 2u, hd.c0, hd.c1);
            step(NR{}, t + 3u, 0u, hd.a0, hd.a1);
        } else {
            if (rem > 0u) step(NR{}, t, 0u, hd.a0, hd.a1);
            if (rem > 1u) step(NR{}, t + 1u, 1u, hd.b0, hd.b1);
            if (rem > 2u) step(NR{}, t + 2u, 2u, hd.c0, hd.c1);
        }
        if (g == 0) sh.oq[pos][n] = acc[0];
    }
}

/* bf16 rounding on the hardware RNE narrow (v_cvt_pk_bf16_f32): the bits
 * of ghip_bf16_round for every finite value, subnormals included, and a
 * quiet NaN for a NaN (the NaNs the combine sees come from the device's
 * own arithmetic, quiet already) */
__device__ __forceinline__ float md_bf16_rnd(float x) {
    return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x) << 16);
}
__device__ __forceinline__ float2 md_bf16_rnd2(float a, float b) {
    typedef __bf16 md_bf2 __attribute__((ext_vector_type(2)));
    typedef float md_f2 __attribute__((ext_vector_type(2)));
    const uint32_t u = __builtin_bit_cast(uint32_t,
                                          __builtin_convertvector((md_f2){a, b}, md_bf2));
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
}

/* y over the first nsel (<= KC) combine positions: every position's output
 * and weight is read before the sum (one LDS round trip; the positions past
 * nsel are left out), the products bf16(bf16(o) * w) are independent, and
 * only the running sum is a chain */
template <int KC>
__device__ __forceinline__ float md_combine_sum(const MdShared &sh, uint32_t nsel,
                                                uint32_t tid) {
    float o[KC], wq[KC];
#pragma unroll
    for (int i = 0; i < KC; i++) {
        o[i] = sh.oq[i][tid];
        wq[i] = sh.wt[i];
    }
    float c[KC];
#pragma unroll
    for (int i = 0; i < KC; i += 2) {
        const float2 eo = md_bf16_rnd2(o[i], o[i + 1]);
        const float2 cc = md_bf16_rnd2(eo.x * wq[i], eo.y * wq[i + 1]);
        c[i] = cc.x;
        c[i + 1] = cc.y;
    }
    float y = 0.0f;
#pragma unroll
    for (int i = 0; i < KC; i++)
        if ((uint32_t)i < nsel) y = md_bf16_rnd(y + c[i]);
    return y;
}

/* the ascending-expert combine of the nsel expert outputs in sh.oq: y =
 * bf16(y + bf16(bf16(o) * w)), from +0 (c/gmoe.h:307-320). Call after a
 * barrier. */
template <bool SHARED>
__device__ __forceinline__ void md_combine(const MdShared &sh, uint32_t r0,
                                           uint16_t *__restrict__ out) {
    const uint32_t tid = threadIdx.x;
    if (tid < 16) {
        const uint32_t nsel = __builtin_amdgcn_readfirstlane(sh.nsel);
        float y = nsel <= 8u ? md_combine_sum<8>(sh, nsel, tid)
                             : md_combine_sum<MD_MAXK>(sh, nsel, tid);
        if constexpr (SHARED) {
            /* the shared expert's output (its waves' partials in wave
             * order, one bf16 rounding), added last with one more rounding
             * and no weight (c/gmoe.h:325-336) */
            float so = sh.sdown[0][tid];
#pragma unroll
            for (uint32_t w = 1; w < MD_NW; w++) so = so + sh.sdown[w][tid];
            y = y + ghip_bf16_round(so);
        }
        out[r0 + tid] = (uint16_t)ghip_bf16_bits(y);
    }
}

/* nw hand-off words (2 nw h values) into LDS (hs32 [nw] words, the bf16
 * pairs as stored) by the calling wave alone, from the words at src (one
 * slot's words, or a range of them): the lanes load their words with
 * device-coherent loads and re-poll the ones that still hold the sentinel
 * (their gate/up item is still running on another CU), at most MD_SPIN_MAX
 * rounds. Returns false (the same in every lane) when a word is still
 * missing then. No workgroup barrier: each wave goes on to its own slot's
 * rows as soon as that slot's h is in. */
__device__ __forceinline__ bool md_stage_h_wave(const uint32_t *src, uint32_t nw,
                                                uint32_t *hs32) {
    constexpr uint32_t PER = 16;
    const uint32_t lane = threadIdx.x & 63u;
    for (uint32_t i0 = 0; i0 < nw; i0 += 64u * PER) {
        uint32_t v[PER];
#pragma unroll
        for (uint32_t u = 0; u < PER; u++) {
            const uint32_t i = i0 + u * 64u + lane;
            v[u] = __hip_atomic_load(src + (i < nw ? i : nw - 1u), __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        }
        /* the wave polls until none of its words is the sentinel (uniform
         * exit) */
        for (uint32_t it = 0;; it++) {
            uint32_t miss = 0;
#pragma unroll
            for (uint32_t u = 0; u < PER; u++) {
                const uint32_t i = i0 + u * 64u + lane;
                miss |= (i < nw && v[u] == MD_HSENT) ? 1u << u : 0u;
            }
            if (!__builtin_amdgcn_readfirstlane((uint32_t)(__ballot(miss != 0u) != 0ull)))
                break;
            if (it >= MD_SPIN_MAX) return false;
            __builtin_amdgcn_s_sleep(4);
#pragma unroll
            for (uint32_t u = 0; u < PER; u++)
                if ((miss >> u) & 1u)
                    v[u] = __hip_atomic_load(src + i0 + u * 64u + lane, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (uint32_t u = 0; u < PER; u++) {
            const uint32_t i = i0 + u * 64u + lane;
            if (i < nw) hs32[i] = v[u];
        }
    }
    return true;
}

/* ------------------------------------------------------------------------ */
/* router with the reference semantics (c/gmoe.h:191-208)                   */
/* ------------------------------------------------------------------------ */

/* Gate logit of one row by one wave: sum_k w[k] * x[k] in f32, lane-strided
 * partial sums (lane l takes k = 8l + 512i, ascending i) and a fixed
 * xor-butterfly reduction: a GEMV of the same tolerance class as every
 * other one here (the reference's sequential-k dot is c/gmoe.h:168-173).
 * Eight row segments per lane are loaded before any is used, so a row
 * costs one memory round trip, not one per segment. dim % 8 == 0, 16-byte
 * aligned rows. */
__device__ __forceinline__ float rt_gate_dot(const uint16_t *__restrict__ row,
                                             const uint16_t *__restrict__ x, uint32_t dim,
                                             uint32_t lane) {
    float acc = 0.0f;
    auto fma8 = [&](const ghip_u32x4 &wv, const ghip_u32x4 &xv) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            acc = acc + __uint_as_float(wv[q] << 16) * __uint_as_float(xv[q] << 16);
            acc = acc + __uint_as_float(wv[q] & 0xffff0000u) *
                            __uint_as_float(xv[q] & 0xffff0000u);
        }
    };
    uint32_t k = lane * 8u;
    for (; k + 7u * 512u < dim; k += 8u * 512u) {
        ghip_u32x4 wv[8], xv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            wv[u] = *(const ghip_u32x4 *)(row + k + 512u * u);
            xv[u] = *(const ghip_u32x4 *)(x + k + 512u * u);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) fma8(wv[u], xv[u]);
    }
    for (; k < dim; k += 512u)
        fma8(*(const ghip_u32x4 *)(row + k), *(const ghip_u32x4 *)(x + k));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = acc + __shfl_xor(acc, off, 64);
    return acc;
}

/* Selection and weights from one wave's logits (c/gmoe.h:191-208): lane l
 * holds the logits lv and biases bv of experts R l .. R l + R - 1 (those
 * past E ignored); scores = numpy-stable sigmoid (device expf), the stable
 * top-k (larger first, ties to the lower id) of score + bias -- the bias
 * selects, it never weighs -- then w_j = score[idx_j] / (pairwise_sum +
 * 1e-20) * route_scale, with numpy's float32 pairwise sum of the k
 * selected scores in selection order (c/gmhc.h:165-185). Lane j < topk
 * returns pick j's id and weight (selection order, as the reference
 * returns them). sc: LDS [E] for the scores; scores (may be NULL): global
 * [E] copy. */
template <int R>
__device__ __forceinline__ void rt_router_core(const float (&lv)[R], const float (&bv)[R],
                                               uint32_t E, int topk, float scale, float *sc,
                                               float *__restrict__ scores, int &myid,
                                               float &myw) {
    const int lane = threadIdx.x & 63;
    uint32_t key[R];
#pragma unroll
    for (int s = 0; s < R; s++) {
        const uint32_t i = (uint32_t)lane * R + s;
        key[s] = 0u;
        if (i < E) {
            const float v = ghip_sigmoid_np(lv[s]);
            sc[i] = v;
            if (scores) scores[i] = v;
            key[s] = rt_key(v + bv[s]);
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);           /* lgkmcnt(0) */
    __builtin_amdgcn_wave_barrier();
    uint32_t mk;
    myid = rt_select<R>(key, topk, mk);
    myw = lane < topk ? sc[myid] : 0.0f;
    /* numpy float32 pairwise sum of the k selected scores (k <= 16) */
    const float myv = myw;
    auto at = [&](int i) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, myv), i));
    };
    float sum;
    if (topk < 8) {
        sum = at(0);
        for (int i = 1; i < topk; i++) sum = sum + at(i);
    } else {
        float r[8];
#pragma unroll
        for (int q = 0; q < 8; q++) r[q] = at(q);
        int i = 8;
        if (topk >= 16) {
#pragma unroll
            for (int q = 0; q < 8; q++) r[q] = r[q] + at(8 + q);
            i = 16;
        }
        sum = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < topk; i++) sum = sum + at(i);
    }
    myw = myv / (sum + 1e-20f) * scale;
}

/* The router's selection from logits read by lg(i) (one wave). */
template <int R, typename Logit>
__device__ __forceinline__ void rt_sigmoid_select(Logit lg, const float *__restrict__ bias,
                                                  uint32_t E, int topk, float scale,
                                                  float *sc, float *__restrict__ scores,
                                                  int32_t *__restrict__ idx,
                                                  float *__restrict__ w) {
    const int lane = threadIdx.x & 63;
    /* logits and biases of all R slots are loaded (clamped index, no
     * predicated load) before any is used: one memory round trip */
    float lv[R], bv[R];
#pragma unroll
    for (int s = 0; s < R; s++) {
        const uint32_t i = (uint32_t)lane * R + s, ic = i < E ? i : E - 1u;
        lv[s] = lg(ic);
        bv[s] = bias[ic];
    }
#pragma unroll
    for (int s = 0; s < R; s++) asm volatile("" ::"v"(lv[s]), "v"(bv[s]));
    int myid;
    float myw;
    rt_router_core<R>(lv, bv, E, topk, scale, sc, scores, myid, myw);
    if (lane < topk) {
        idx[lane] = myid;
        w[lane] = myw;
    }
}

/* Phase A of the router-fed decode, wave 0 of every workgroup: the gate
 * logits of all E experts, published by the workgroups that computed them
 * as 64-bit words (this launch's tag in bits 32..47, the f32 logit in
 * 0..31; device-coherent stores and loads, as the h hand-off), polled until
 * each carries the tag (bounded: on a run-out nothing is selected and
 * err |= 4), then the reference router's selection and weights
 * (rt_router_core): sel in selection order, wt at the ascending-id combine
 * positions. Workgroup 0 also writes the picks to
 * idx_out / w_out when given. sc: LDS [E]. */
template <int R>
__device__ __forceinline__ void md_route_router(const uint64_t *lw, const float *__restrict__ bias,
                                                uint32_t E, int topk, float scale,
                                                uint32_t tag, float *sc, MdShared &sh,
                                                uint32_t *__restrict__ err,
                                                int32_t *__restrict__ idx_out,
                                                float *__restrict__ w_out) {
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t v[R];
    float bv[R];
#pragma unroll
    for (int s = 0; s < R; s++) {
        const uint32_t i = lane * R + s, ic = i < E ? i : E - 1u;
        v[s] = __hip_atomic_load(lw + ic, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bv[s] = bias[ic];
    }
    for (uint32_t it = 0;; it++) {
        uint32_t miss = 0;
#pragma unroll
        for (int s = 0; s < R; s++)
            miss |= (lane * R + s < E && (uint32_t)(v[s] >> 32) != tag) ? 1u << s : 0u;
        if (!__builtin_amdgcn_readfirstlane((uint32_t)(__ballot(miss != 0u) != 0ull))) break;
        if (it >= MD_SPIN_MAX) {
            if (lane == 0) {
                sh.nsel = 0;
                atomicOr(err, 4u);
            }
            return;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int s = 0; s < R; s++)
            if ((miss >> s) & 1u)
                v[s] = __hip_atomic_load(lw + lane * R + s, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    }
    float lv[R];
#pragma unroll
    for (int s = 0; s < R; s++) lv[s] = __uint_as_float((uint32_t)v[s]);
    int myid;
    float myw;
    rt_router_core<R>(lv, bv, E, topk, scale, sc, nullptr, myid, myw);
    const int id_or_max = (int)lane < topk ? myid : 0x7fffffff;
    int rank = 0;
    for (int j = 0; j < topk; j++) rank += __builtin_amdgcn_readlane(id_or_max, j) < id_or_max;
    if ((int)lane < topk) {
        sh.sel[lane] = myid;
        sh.wt[rank] = myw;
        if (idx_out && blockIdx.x == 0) {
            idx_out[lane] = myid;
            w_out[lane] = myw;
        }
    }
    if (lane == 0) sh.nsel = (uint32_t)topk;
}

/* ------------------------------------------------------------------------ */
/* the decode launch                                                        */
/* ------------------------------------------------------------------------ */

/* One launch of gridDim.x workgroups (one per CU), 8 waves each. hw: this
 * launch's h words ([max topk + 1][inter / 2] u32, two bf16 per word), all
 * MD_HSENT when the launch starts; hw_clr: the other buffer (clr_words
 * words), which the launch refills with MD_HSENT for the next one (the
 * launch before this one read it, and stream order has it done). tag:
 * this launch's tag for the router's logit words (1..65535; the host
 * clears those whenever the tag wraps, so no stale word carries a live
 * tag). The hand-off needs every workgroup resident at once: the grid
 * is one workgroup per CU, which an otherwise idle device always holds.
 * When other work holds CUs, a workgroup may wait for a slot while the
 * resident ones wait for its h: a wait for h that runs out (MD_SPIN_MAX
 * polls) flags err |= 4 and that wave skips its down rows (in every later
 * row group too) instead of hanging, so the launch always ends, and its
 * output is invalid whenever the word holds 4 afterwards. */
/* The reference router's inputs and outputs for the router-fed decode. */
struct MdRouter {
    const uint16_t *gate_w;      /* [E, dim] bf16 */
    const float *bias;           /* [E] f32, selection only */
    float scale;                 /* route_scale (routed_scaling_factor) */
    uint64_t *lw;                /* [E] tagged logit words (workspace) */
    int32_t *idx_out;            /* [topk] or NULL */
    float *w_out;                /* [topk] or NULL */
};

/* The arguments the routing phase needs come first, so they arrive with the
 * kernel's first kernel-argument loads and the logits and x loads wait for
 * one round of them, not two; n_experts and dim repeat bank's. */
template <bool SHARED, bool ROUTER>
__global__ __launch_bounds__(MD_NW * 64, 1) void k_moe_decode(
    const float *__restrict__ logits, const uint16_t *__restrict__ x,
    const int32_t *__restrict__ idx, const float *__restrict__ w,
    uint32_t *__restrict__ err, int topk, uint32_t n_experts, uint32_t dim,
    GhipBank bank, float limit, uint32_t *hw, uint32_t *hw_clr, uint32_t clr_words,
    uint32_t tag, uint16_t *__restrict__ out, MdRouter rtr) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t dl[];
    __shared__ MdShared sh;
    const uint32_t tid = threadIdx.x;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t inter = bank.inter;
    uint16_t *xs = (uint16_t *)dl;
    uint8_t *gu_ring = dl + ((dim * 2u + 1023u) & ~1023u);

    /* --- phase A: route (wave 0) while x goes to LDS ------------------- */
    {
        /* the first MD_NW * 64 pieces of x are loaded before the routing, so
         * the routing wave's piece does not cost a round trip after it */
        const uint32_t n16 = dim >> 3;
        const ghip_u32x4 x0 = ((const ghip_u32x4 *)x)[tid < n16 ? tid : n16 - 1];
        if constexpr (ROUTER) {
            /* the gate logits: wave v of workgroup b computes expert
             * b + v * G's, published as a tagged word (c/gmoe.h:168-173) */
            const uint32_t r = blockIdx.x + wv * gridDim.x;
            if (r < n_experts) {
                const float acc = rt_gate_dot(rtr.gate_w + (size_t)r * dim, x, dim, tid & 63u);
                if ((tid & 63u) == 0)
                    __hip_atomic_store(rtr.lw + r, ((uint64_t)tag << 32) | __float_as_uint(acc),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (wv == 0) {
            if constexpr (ROUTER) {
                float *rsc = (float *)gu_ring;            /* wave 0's area: idle in phase A */
                if (n_experts <= 5 * 64)
                    md_route_router<5>(rtr.lw, rtr.bias, n_experts, topk, rtr.scale, tag,
                                       rsc, sh, err, rtr.idx_out, rtr.w_out);
                else
                    md_route_router<8>(rtr.lw, rtr.bias, n_experts, topk, rtr.scale, tag,
                                       rsc, sh, err, rtr.idx_out, rtr.w_out);
            } else {
                md_route_ids(logits, idx, w, topk, (int)n_experts, sh,
                             blockIdx.x == 0 ? err : nullptr);
            }
        } else if (SHARED && blockIdx.x * 8u < inter)
            /* the other waves stream the shared expert's gate/up rows of
             * this workgroup meanwhile (no routing needed) */
            md_shared_gateup(bank, x, gu_ring + wv * (GU_R * GU_STG), blockIdx.x, sh);
        asm volatile("" ::"v"(x0));
        if (tid < n16) ((ghip_u32x4 *)xs)[tid] = x0;
        for (uint32_t i = tid + MD_NW * 64; i < n16; i += MD_NW * 64)
            ((ghip_u32x4 *)xs)[i] = ((const ghip_u32x4 *)x)[i];
        /* nothing of the routing (its error-flag atomic included) stays in
         * flight into the streaming loops */
        GHIP_VMCNT(0);
        __syncthreads();
        if (SHARED && wv == 1 && blockIdx.x * 8u < inter)
            md_shared_h(sh, blockIdx.x, inter, limit, hw);
    }

    /* the other h buffer back to the sentinel for the next launch (at most
     * one word per thread at the model's shapes; its store latency joins
     * the first gate/up stage's wait) */
    for (uint32_t i = blockIdx.x * (MD_NW * 64u) + tid; i < clr_words;
         i += gridDim.x * (MD_NW * 64u))
        __hip_atomic_store(hw_clr + i, MD_HSENT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    /* --- phase B: gate/up + SwiGLU -> h hand-off words ------------------ */
    md_phase_gateup(bank, xs, gu_ring, sh, limit, hw);

    /* --- phase C: down + combine per 16 output rows -------------------- */
    const uint32_t nsel = __builtin_amdgcn_readfirstlane(sh.nsel);
    uint16_t *hs = (uint16_t *)dl;
    uint8_t *ring = dl + (size_t)MD_NW * inter * 2u;
    if (!ROUTER && wv == 0 && logits) md_route_finish(sh, topk);
    /* whether this wave's staged h is this launch's (false once a wait ran
     * out: the wave then computes no down rows at all, in this row group
     * or in a later one that reuses the staged h) */
    bool hs_ok = true;
    /* shared expert: wave w's share of inter, k blocks [sc0, sc1), and its
     * h values staged once at hss (after the down rings) */
    const uint32_t nchd = inter >> 7;
    const uint32_t sc0 = wv * nchd / MD_NW, sc1 = (wv + 1u) * nchd / MD_NW;
    uint16_t *hss = (uint16_t *)(ring + (size_t)MD_NW * DN_R * DN_STG) + wv * (nchd / MD_NW + 1u) * 128u;
    bool hss_ok = true;
    for (uint32_t rg = blockIdx.x; rg * MD_T < dim; rg += gridDim.x) {
        const uint32_t r0 = rg * MD_T;
        if constexpr (SHARED) {
            /* the shared expert's down rows over this wave's share of
             * inter, while the routed slots' h is still on its way */
            if (rg == blockIdx.x && sc1 > sc0)
                hss_ok = md_stage_h_wave(hw + (size_t)MD_SH_SLOT * (inter / 2u) + sc0 * 64u,
                                         (sc1 - sc0) * 64u, (uint32_t *)hss);
            ghip_f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
            if (hss_ok && sc1 > sc0) {
                const uint32_t nkb = inter >> 7;
                const uint8_t *slab = bank.base + (size_t)bank.n_experts * bank.stride;
                const uint8_t *rows = slab + bank.off_dw + (size_t)r0 * inter;
                const float *srow = (const float *)(slab + bank.off_ds) + (size_t)(r0 >> 7) * nkb;
                const ghip_cdma d = ghip_cdma_offsets(tid & 63u, inter);
                uint8_t *wring = ring + wv * (DN_R * DN_STG);
                if (ghip_sload_u32(bank.nan_flags, bank.n_experts) != 0u)
                    md_shared_down_blocks<true>(rows, srow, hss, d, sc0, sc1, wring, sacc);
                else
                    md_shared_down_blocks<false>(rows, srow, hss, d, sc0, sc1, wring, sacc);
            } else if (!hss_ok && (tid & 63u) == 0) {
                atomicOr(err, 4u);
            }
            if ((tid & 63u) < 16u) sh.sdown[wv][tid & 63u] = sacc[0];
        }
        for (uint32_t base = 0; base < nsel; base += MD_NW) {
            /* the down rows' first chunks stream while h is awaited */
            MdDownHead hd = md_down_prologue(bank, sh, r0, base);
            /* wave w: h of slot base + w (once when all slots fit one
             * pass), then at once its down rows; a wave whose wait runs
             * out flags the error and computes nothing */
            if (base + wv < nsel && (base > 0 || rg == blockIdx.x || nsel > MD_NW))
                hs_ok = md_stage_h_wave(hw + (size_t)(base + wv) * (inter / 2u), inter / 2u,
                                        (uint32_t *)(hs + (size_t)wv * inter));
            const bool ok = hs_ok;
            if (ok) {
                md_phase_down(bank, sh, r0, base, hs, ring, hd);
            } else {
                if ((tid & 63u) == 0) atomicOr(err, 4u);
                GHIP_VMCNT(0);                    /* drain the chunk loads */
            }
            __syncthreads();
        }
        if (SHARED && nsel == 0) __syncthreads();  /* the shared partials are in */
        md_combine<SHARED>(sh, r0, out);
        __syncthreads();                          /* sh.oq is reused by the next rows */
    }
}

/* The whole router in one launch: workgroup b's waves compute gate logits
 * 4b..4b+3 and store them with agent-scope (device-coherent) stores; each
 * workgroup waits for its stores, then bumps a counter with an agent-scope
 * release; the workgroup that arrives last takes an agent-scope acquire,
 * resets the counter and selects from the logits (read with agent-scope
 * loads, so logits written on other XCDs are seen), with no second
 * launch. The counter starts at 0 and every launch
 * leaves it at 0; launches that overlap on one device race. */
__global__ __launch_bounds__(256) void k_router(const uint16_t *__restrict__ gate_w,
                                                const uint16_t *__restrict__ x, uint32_t E,
                                                uint32_t dim, const float *__restrict__ bias,
                                                int topk, float scale, float *logits_ws,
                                                uint32_t *count, float *__restrict__ scores,
                                                int32_t *__restrict__ idx,
                                                float *__restrict__ w) {
    __shared__ float sc[RT_MAXE];
    __shared__ uint32_t last;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, e = blockIdx.x * 4u + (tid >> 6);
    if (e < E) {
        const float acc = rt_gate_dot(gate_w + (size_t)e * dim, x, dim, lane);
        if (lane == 0)
            __hip_atomic_store((uint32_t *)logits_ws + e, __float_as_uint(acc),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    GHIP_VMCNT(0);                                /* own logit stores complete */
    __syncthreads();
    /* the arrival is a release (this workgroup's logit stores happen
     * before it); the last workgroup acquires before reading the logits */
    if (tid == 0)
        last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT)
               == gridDim.x - 1;
    __syncthreads();
    if (!last || tid >= 64) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    auto lg = [&](uint32_t i) {
        return __uint_as_float(__hip_atomic_load((const uint32_t *)logits_ws + i,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    };
    if (E <= 5 * 64) rt_sigmoid_select<5>(lg, bias, E, topk, scale, sc, scores, idx, w);
    else rt_sigmoid_select<8>(lg, bias, E, topk, scale, sc, scores, idx, w);
}

/* Selection from given logits (one wave). */
__global__ __launch_bounds__(64) void k_router_select(const float *__restrict__ logits,
                                                      const float *__restrict__ bias,
                                                      uint32_t E, int topk, float scale,
                                                      float *__restrict__ scores,
                                                      int32_t *__restrict__ idx,
                                                      float *__restrict__ w) {
    __shared__ float sc[RT_MAXE];
    auto lg = [&](uint32_t i) { return logits[i]; };
    if (E <= 5 * 64) rt_sigmoid_select<5>(lg, bias, E, topk, scale, sc, scores, idx, w);
    else rt_sigmoid_select<8>(lg, bias, E, topk, scale, sc, scores, idx, w);
}

extern "C" hipError_t ghip_launch_moe_router(const uint16_t *x, const uint16_t *gate_w,
                                             const float *logits_in, float *logits_ws,
                                             uint32_t *count, const float *bias, uint32_t E,
                                             uint32_t dim, int topk, float scale,
                                             float *scores, int32_t *idx, float *w,
                                             const hipEvent_t *ev, hipStream_t st) {
    if (!bias || !idx || !w || E == 0 || E > RT_MAXE || topk <= 0 || topk > MD_MAXK
        || (uint32_t)topk > E)
        return hipErrorInvalidValue;
    hipEvent_t ev0 = ev ? ev[0] : nullptr, ev1 = ev ? ev[1] : nullptr;
    if (!logits_in) {
        if (!x || !gate_w || !logits_ws || !count || dim == 0 || dim % 8
            || ((uintptr_t)x & 15) || ((uintptr_t)gate_w & 15))
            return hipErrorInvalidValue;
        GHIP_LAUNCH(ev0, ev1, k_router, dim3((E + 3) / 4), dim3(256), 0, st, gate_w, x, E, dim,
                    bias, topk, scale, logits_ws, count, scores, idx, w);
        return hipGetLastError();
    }
    GHIP_LAUNCH(ev0, ev1, k_router_select, dim3(1), dim3(64), 0, st, logits_in, bias, E,
                topk, scale, scores, idx, w);
    return hipGetLastError();
}

extern "C" hipError_t ghip_launch_moe_decode(const GhipBank *bank,
                                             const uint16_t *x,
                                             const float *logits,
                                             const int32_t *idx, const float *w,
                                             const GhipRouterArgs *router,
                                             int topk, float limit,
                                             uint16_t *out,
                                             GhipMoeDecodeWs *ws,
                                             const hipEvent_t *ev,
                                             hipStream_t st) {
    if (!bank || !bank->nan_flags || !ws || !x || !out) return hipErrorInvalidValue;
    const uint32_t dim = bank->dim, inter = bank->inter;
    if (topk <= 0 || topk > MD_MAXK || (uint32_t)topk > bank->n_experts)
        return hipErrorInvalidValue;
    if (!router && !logits && (!idx || !w)) return hipErrorInvalidValue;
    if (dim == 0 || inter == 0 || dim % 128 || inter % 128) return hipErrorInvalidValue;
    if ((logits || router) && bank->n_experts > RT_MAXE) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) || ((uintptr_t)bank->base & 15) || (bank->stride & 15)
        || (bank->off_gw & 15) || (bank->off_uw & 15) || (bank->off_dw & 15)
        || (bank->off_gs & 3) || (bank->off_us & 3) || (bank->off_ds & 3))
        return hipErrorInvalidValue;
    MdRouter rtr = {nullptr, nullptr, 0.0f, nullptr, nullptr, nullptr};
    if (router) {
        /* the gate rows go one to a wave, at most MD_NW per workgroup */
        if (!router->gate_w || !router->bias || !ws->lw || ((uintptr_t)router->gate_w & 15)
            || (size_t)bank->n_experts > (size_t)MD_NW * ws->n_cu
            || (!router->idx_out) != (!router->w_out))
            return hipErrorInvalidValue;
        rtr = {router->gate_w, router->bias, router->route_scale, ws->lw, router->idx_out,
               router->w_out};
    }
    const bool shared = bank->has_shared != 0;
    const size_t lds_gu = (((size_t)dim * 2 + 1023) & ~(size_t)1023) + GU_NW * GU_R * GU_STG;
    /* down: the slots' h, the chunk rings and, with a shared expert, each
     * wave's share of its h */
    const size_t lds_dn = (size_t)MD_NW * inter * 2 + MD_NW * DN_R * DN_STG
                        + (shared ? (size_t)MD_NW * (inter / 128 / MD_NW + 1) * 256 : 0);
    const size_t lds = lds_gu > lds_dn ? lds_gu : lds_dn;
    if (lds > MD_LDS_MAX || ws->n_cu == 0 || !ws->hw || !ws->err || inter > ws->hw_inter)
        return hipErrorInvalidValue;
    /* the shared expert's gate/up rows go 8 to a workgroup, in one pass */
    if (shared && (size_t)inter > (size_t)ws->n_cu * 8) return hipErrorInvalidValue;
    /* the tag and the h buffer parity are host state advanced per call, so
     * a launch recorded into a graph would replay with stale ones: refuse
     * to be captured */
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return hipErrorStreamCaptureUnsupported;
    /* one workgroup per CU (the LDS use keeps it at one); the tag names
     * this launch's logit words: 1..65535, and when it wraps the words are
     * cleared first (by a fill kernel, ordered on st), so a word left from
     * 65535 launches ago cannot pass for this launch's. The h words need
     * no tag: the launch writes buffer ws->hpar, which holds only the
     * sentinel, and refills the other one. */
    hipError_t e;
    if (++ws->tag > 0xffffu) {
        if (ws->lw && (e = ghip_launch_fill_u32((uint32_t *)ws->lw, 2 * (size_t)RT_MAXE, 0u,
                                                st)) != hipSuccess)
            return e;
        ws->tag = 1;
    }
    const size_t hbuf = (size_t)(MD_MAXK + 1) * (ws->hw_inter / 2u);
    uint32_t *hcur = ws->hw + (ws->hpar ? hbuf : 0), *hclr = ws->hw + (ws->hpar ? 0 : hbuf);
    hipEvent_t e0 = ev ? ev[0] : nullptr, e1 = ev ? ev[1] : nullptr;
    const dim3 grid(ws->n_cu), blk(MD_NW * 64);
#define MD_LAUNCH(S, R_)                                                               \
    GHIP_LAUNCH(e0, e1, (k_moe_decode<S, R_>), grid, blk, lds, st, logits, x, idx, w, ws->err, \
                topk, bank->n_experts, bank->dim, *bank, limit, hcur, hclr, (uint32_t)hbuf,    \
                ws->tag, out, rtr)
    if (shared) {
        if (router) MD_LAUNCH(true, true);
        else MD_LAUNCH(true, false);
    } else {
        if (router) MD_LAUNCH(false, true);
        else MD_LAUNCH(false, false);
    }
#undef MD_LAUNCH
    /* the next launch writes the buffer this one refills (only once this
     * one is enqueued: a launch that never ran refilled nothing) */
    if ((e = hipGetLastError()) == hipSuccess) ws->hpar ^= 1u;
    return e;
}

extern "C" hipError_t ghip_moe_decode_init(void) {
    const void *k[4] = {(const void *)k_moe_decode<false, false>,
                        (const void *)k_moe_decode<false, true>,
                        (const void *)k_moe_decode<true, false>,
                        (const void *)k_moe_decode<true, true>};
    for (int i = 0; i < 4; i++) {
        hipError_t e = hipFuncSetAttribute(k[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                           MD_LDS_MAX);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
