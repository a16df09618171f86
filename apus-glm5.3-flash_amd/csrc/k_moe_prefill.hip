/*
 * k_moe_prefill.hip — K4: routed-MoE prefill for T tokens on gfx950.
 *
 * The reference has no grouped GEMM: its prefill runs, per token, the
 * selected experts' three GEMVs and the ordered combine (c/gmoe.h:278-320,
 * expert body c/gmoe.h:210-227). Here the same result is computed as
 * grouped GEMMs over expert-sorted (token, expert) pairs:
 *
 *   k_pf_count    pairs -> per-chunk expert histogram; validates ids and
 *                 drops repeated ids of a token (the reference loop uses the
 *                 first slot that names an expert, c/gmoe.h:309-311).
 *   k_pf_scan     one workgroup: exclusive offsets per (chunk, expert), the
 *                 expert-sorted row ranges and the tile list.
 *   k_pf_scatter  stable scatter (token order inside each expert).
 *   k_pf_gemm<0, NW>  gate/up: H[s] = SwiGLU(bf16(x Wg^T), bf16(x Wu^T)) for the
 *                 sorted pair rows s of each tile; x rows gathered by token.
 *   k_pf_gemm<1, NW>  down: O[s] = bf16(H[s] Wd^T).
 *   k_pf_combine  out[t] = ascending-expert, bf16-per-add sum of
 *                 bf16(O[s] * w) over the token's pairs (c/gmoe.h:307-320).
 *
 * GEMM tile (both modes). A workgroup of 4 waves (NW = 4) owns one tile of
 * up to 256 expert-sorted rows and one column block; K is walked in
 * 64-wide stages (half an F32 scale block). Each wave owns two 32-column
 * weight slots (gate and up columns [c, c+32) in mode 0, so the SwiGLU
 * epilogue is lane-local; two 128-apart down column groups in mode 1) for
 * all tile rows, accumulating 2 x NRB v_mfma_f32_32x32x16_bf16 blocks.
 * With NW = 8 (two waves per SIMD) the same tile is split into two row
 * halves, so one wave's MFMAs run while the other issues its DMA. Both
 * operands stream HBM -> LDS by direct DMA (global_load_lds) through a ring
 * of stages, the activation rows gathered by token in mode 0; the FP8 codes
 * are dequantized in registers when read from LDS, bit-exact
 * (bf16_rne(e4m3 * scale), c/fp8blk.h:115-136). MFMA step s of lane half h
 * takes k = 32h + 8s + [0, 8) of the stage from both operands. 32-row blocks
 * past the tile's row count are neither loaded nor computed, so ragged
 * experts cost what their rows need.
 *
 * The GEMM grid is persistent and XCD-aware: one workgroup per CU;
 * hardware deals workgroups to the 8 XCDs round-robin, so workgroup b
 * (XCD b % 8) works on tiles b % 8, b % 8 + 8, ... and the XCD's
 * workgroups split each tile's column blocks: the column blocks of one tile
 * (same gathered activation rows) run on one XCD and share its L2, and the
 * worst-case tile count sizes nothing (the real count is read on the
 * device).
 */
#include "ghip_device.h"
#include "ghip_internal.h"

#include <type_traits>

typedef float ghip_f32x16 __attribute__((ext_vector_type(16)));

#define PF_CHUNK 1024            /* pairs per permutation workgroup */
#define PF_BM 256                /* rows per GEMM tile */
#define PF_RB (PF_BM / 32)       /* 32-row MFMA blocks per tile */
#define PF_BK 64                 /* k per pipeline stage */
#define PF_A_STAGE (PF_BM * PF_BK * 2)          /* 32 KB activation tile */
#define PF_W_STAGE (256 * PF_BK)                /* 16 KB FP8 weight rows */
#define PF_STAGE (PF_A_STAGE + PF_W_STAGE)
#define PF_RING (3 * PF_STAGE)                  /* 144 KB ring */
#define PF_SCT_MAX 128           /* k blocks in the per-tile scale table (K <= 16384) */
#define PF_LDS (PF_RING + PF_SCT_MAX * 8)       /* ring + scale table */
#define PF_WB (256 * 128)                       /* 32 KB weight block: 256 rows x 128 k */
#define PF_LDS_WB (3 * PF_A_STAGE + 2 * PF_WB)  /* the full-tile 8-wave body: 160 KB */
#define PF_MAXK 16               /* max top-k per token */
#define PF_MAXE 1024             /* max experts in a bank */

/* ------------------------------------------------------------------------ */
/* permutation                                                              */
/* ------------------------------------------------------------------------ */

/* One workgroup per PF_CHUNK pairs. A token has topk_p = topk + shared
 * pair slots: pair p = t * topk_p + j is (token t, idx[t * topk + j]) for
 * j < topk, and (token t, the shared expert, id E) for j == topk when the
 * bank has one (c/gmoe.h:325-336: every token runs it). eid[p] = the expert
 * of p, or -1 when a routed id is out of range (flags hdr[PF_HDR_ERR] and,
 * when given, bit 2 of the store's sticky error word serr) or repeats an
 * earlier slot of the same token. cnt[chunk][e] = count (E + shared
 * experts). */
__global__ __launch_bounds__(1024) void k_pf_count(
    const int32_t *__restrict__ idx, uint32_t P, uint32_t topk, uint32_t topk_p,
    uint32_t E, uint32_t *__restrict__ cnt, int32_t *__restrict__ eid,
    uint32_t *__restrict__ hdr, uint32_t *__restrict__ serr) {
    extern __shared__ uint32_t hist[];
    const uint32_t Ep = E + (topk_p - topk);
    for (uint32_t i = threadIdx.x; i < Ep; i += 1024) hist[i] = 0;
    __syncthreads();
    const uint32_t p = blockIdx.x * PF_CHUNK + threadIdx.x;
    if (p < P) {
        const uint32_t t = p / topk_p, j = p - t * topk_p;
        const int32_t e = j < topk ? idx[(size_t)t * topk + j] : (int32_t)E;
        bool ok = e >= 0 && (uint32_t)e < Ep;
        if (!ok || (j < topk && (uint32_t)e == E)) {
            ok = false;
            atomicOr(&hdr[PF_HDR_ERR], 1u);
            if (serr) atomicOr(serr, 2u);
        } else if (j < topk) {
            for (uint32_t jj = 0; jj < j; jj++)
                if (idx[(size_t)t * topk + jj] == e) { ok = false; break; }
        }
        eid[p] = ok ? e : -1;
        if (ok) atomicAdd(&hist[e], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < Ep; i += 1024)
        cnt[(size_t)blockIdx.x * Ep + i] = hist[i];
}

/* Inclusive scan of one value per thread over a 1024-thread workgroup. */
__device__ __forceinline__ uint32_t pf_block_scan(uint32_t v, uint32_t *sh) {
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = __shfl_up(v, d, 64);
        if (lane >= (uint32_t)d) v += o;
    }
    if (lane == 63) sh[w] = v;
    __syncthreads();
    if (w == 0) {
        uint32_t s = lane < 16 ? sh[lane] : 0;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            uint32_t o = __shfl_up(s, d, 64);
            if (lane >= (uint32_t)d) s += o;
        }
        if (lane < 16) sh[lane] = s;
    }
    __syncthreads();
    const uint32_t r = v + (w ? sh[w - 1] : 0);
    __syncthreads();
    return r;
}

/* One workgroup of 1024 threads, thread e = expert e. cnt becomes the
 * exclusive start offset (in the expert-sorted order) of each (chunk,
 * expert); tiles[] = {expert, first sorted row, rows, NaN-code flag of the
 * expert (nan_flags[e] != 0; 0 without nan_flags)}; hdr gets the tile
 * count and the number of valid pairs. */
__global__ __launch_bounds__(1024) void k_pf_scan(
    uint32_t *__restrict__ cnt, uint32_t nch, uint32_t E,
    const uint32_t *__restrict__ nan_flags,
    uint4 *__restrict__ tiles, uint32_t *__restrict__ hdr) {
    __shared__ uint32_t sh[16];
    const uint32_t e = threadIdx.x;
    /* the chunk counts are read in batches of 16 independent loads (one
     * memory round trip per batch, not per chunk): a total pass, then the
     * block scan, then a pass that writes each chunk's start row */
    uint32_t tot = 0;
    if (e < E)
        for (uint32_t c0 = 0; c0 < nch; c0 += 16) {
            uint32_t v[16];
#pragma unroll
            for (uint32_t u = 0; u < 16; u++)
                v[u] = c0 + u < nch ? cnt[(size_t)(c0 + u) * E + e] : 0u;
#pragma unroll
            for (uint32_t u = 0; u < 16; u++) tot += v[u];
        }
    const uint32_t nt = (tot + PF_BM - 1) / PF_BM;
    const uint32_t base = pf_block_scan(tot, sh) - tot;
    const uint32_t tb = pf_block_scan(nt, sh) - nt;
    if (e < E) {
        const uint32_t nanf = nan_flags && nan_flags[e] ? 1u : 0u;
        uint32_t run = base;
        for (uint32_t c0 = 0; c0 < nch; c0 += 16) {
            uint32_t v[16];
#pragma unroll
            for (uint32_t u = 0; u < 16; u++)
                v[u] = c0 + u < nch ? cnt[(size_t)(c0 + u) * E + e] : 0u;
#pragma unroll
            for (uint32_t u = 0; u < 16; u++)
                if (c0 + u < nch) {
                    cnt[(size_t)(c0 + u) * E + e] = run;
                    run += v[u];
                }
        }
        for (uint32_t i = 0; i < nt; i++) {
            const uint32_t r0 = i * PF_BM;
            const uint32_t rows = tot - r0 < PF_BM ? tot - r0 : PF_BM;
            tiles[tb + i] = make_uint4(e, base + r0, rows, nanf);
        }
    }
    if (e == 1023) {
        hdr[PF_HDR_NTILES] = tb + nt;
        hdr[PF_HDR_NPAIRS] = base + tot;
    }
}

/* Stable scatter: pair p of chunk c goes to sorted row
 * cnt[c][e] + (earlier pairs of the chunk with expert e). Inside a wave
 * the rank comes from ballots over each distinct expert id (wave-uniform
 * loop); across the chunk's 16 waves from per-wave counts in LDS. */
__global__ __launch_bounds__(1024) void k_pf_scatter(
    const int32_t *__restrict__ eid, uint32_t P, uint32_t E,
    const uint32_t *__restrict__ cnt, int32_t *__restrict__ perm,
    int32_t *__restrict__ pos) {
    extern __shared__ uint32_t wcnt[];                  /* [16][E] */
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (uint32_t i = threadIdx.x; i < 16 * E; i += 1024) wcnt[i] = 0;
    __syncthreads();
    const uint32_t p = blockIdx.x * PF_CHUNK + threadIdx.x;
    const int32_t e = p < P ? eid[p] : -1;
    uint32_t rank = 0;
    uint64_t todo = __ballot(e >= 0);
    while (todo) {
        const int lead = __builtin_ctzll(todo);
        const int32_t e0 = __builtin_amdgcn_readlane(e, lead);
        const uint64_t m = __ballot(e == e0);
        if (e == e0) rank = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == (uint32_t)lead) wcnt[w * E + e0] = __popcll(m);
        todo &= ~m;
    }
    __syncthreads();
    if (e >= 0) {
        for (uint32_t w2 = 0; w2 < w; w2++) rank += wcnt[w2 * E + e];
        const uint32_t s = cnt[(size_t)blockIdx.x * E + e] + rank;
        perm[s] = (int32_t)p;
        pos[p] = (int32_t)s;
    } else if (p < P) {
        pos[p] = -1;
    }
}

/* ------------------------------------------------------------------------ */
/* grouped GEMM                                                             */
/* ------------------------------------------------------------------------ */

/* SwiGLU of the prefill epilogue: the clamp order and bf16 roundings of
 * c/gmoe.h:217-225 with the numpy-stable sigmoid (c/gmhc.h:157-160) on the
 * hardware exp2 and reciprocal. Their f32 results may differ from libm's
 * expf and an IEEE division by an ulp, but the bf16 value bf16(g * s(g))
 * that follows does not: it is a function of the bf16 gate alone, and on
 * all 65,536 gate values it equals the reference's (an exhaustive device
 * test at the model's clamp limit). */
__device__ __forceinline__ uint16_t pf_bf16_bits(float x) {
    /* the hardware RNE narrow (v_cvt_pk_bf16_f32): the reference's bits for
     * every finite value, subnormals included, and a quiet NaN for a NaN */
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ float pf_bf16_round(float x) {
    return __uint_as_float((uint32_t)pf_bf16_bits(x) << 16);
}

/* pf_bf16_round of two values with one packed convert */
__device__ __forceinline__ float2 pf_bf16_round2(float a, float b) {
    typedef __bf16 pf_bf2 __attribute__((ext_vector_type(2)));
    typedef float pf_f2 __attribute__((ext_vector_type(2)));
    const pf_bf2 h = __builtin_convertvector((pf_f2){a, b}, pf_bf2);
    const uint32_t u = __builtin_bit_cast(uint32_t, h);
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
}

/* SwiGLU of the fp32 gate / up accumulators: each rounded to bf16 first,
 * then the clamps (compares, so a NaN stays NaN as in the reference) */
__device__ __forceinline__ uint16_t pf_swiglu(float accg, float accu, float limit) {
    float g = pf_bf16_round(accg), u = pf_bf16_round(accu);
    /* selects, not branches: an if/else chain compiles to exec-mask
     * branches around every element of the epilogue */
    g = g > limit ? limit : g;
    u = u > limit ? limit : (u < -limit ? -limit : u);
    /* e = exp(-|g|) on the hardware exp2 (v_exp_f32), which flushes results
     * below 2^-126 to zero: there (|g| > ~87.3, e subnormal as in libm's
     * expf) the argument is raised by 64 (exactly: both have exponent >= 6)
     * and the result scaled back by 2^-64, one rounding onto the subnormal
     * grid. Over all 65,536 bf16 gate values the resulting h equals the
     * one computed with the host's libm expf (checked exhaustively on the
     * device against the oracle). */
    const float y = -fabsf(g) * 1.44269504088896341f;
    const bool tiny = y < -126.0f;
    const float e = __builtin_amdgcn_exp2f(tiny ? y + 64.0f : y) * (tiny ? 0x1p-64f : 1.0f);
    /* 1 / (1 + e) for 1 + e in (1, 2]: the hardware reciprocal (1 ulp) and
     * one Newton step with fused multiply-adds, which lands on the
     * correctly rounded value (the IEEE division sequence costs ~10
     * instructions per element of the epilogue) */
    const float d = 1.0f + e;
    const float r0 = __builtin_amdgcn_rcpf(d);
    const float r = __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
    const float sg = g >= 0.0f ? r : e * r;
    return pf_bf16_bits(pf_bf16_round(g * sg) * u);
}

/* 8 codes (two dwords) -> one bf16x8 MFMA operand. */
template <bool EXACT>
__device__ __forceinline__ ghip_bf16x8 pf_deq8(uint32_t d0, uint32_t d1, float s) {
    ghip_u32x2 a = ghip_deq4<EXACT>(d0, s), b = ghip_deq4<EXACT>(d1, s);
    ghip_u32x4 v = {a[0], a[1], b[0], b[1]};
    return __builtin_bit_cast(ghip_bf16x8, v);
}

/* What one workgroup computes (see k_pf_gemm). */
struct PfTile {
    const uint16_t *act;          /* activation matrix (x or H), K wide */
    const int32_t *perm;          /* sorted row -> pair (mode 0 gather) */
    const uint8_t *w0, *w1;       /* weight matrices of the two slots */
    const float *sr0, *sr1;       /* scale rows of the two slots */
    uint16_t *out;
    float *outf;                  /* MODE 2: fp32 partial outputs */
    uint32_t K, KS, N, row0, rows, cb0, cb1, topk;  /* cbX: slot X column base */
    float limit;                  /* K: row stride; KS: k span of this tile */
};

/* The tile body for tiles of at most NRB 32-row blocks (rows past NRB*32
 * are neither loaded nor computed; rows past `rows` inside the last block
 * repeat the last row: computed, never stored).
 *
 * K advances in stages of 64 through an NS-deep LDS ring filled by direct
 * global->LDS loads (no register staging). Stage layout, 16-byte pieces
 * XOR-swizzled so the MFMA operand reads hit distinct banks:
 *   A  [NRB*32 rows][8 pieces]  piece p of row r at (p ^ ((r >> 1) & 7))
 *   W  [256 rows][4 pieces]     weight row wr = 64*wave + 32*slot + n,
 *                               piece p at (p ^ ((wr >> 2) & 3))
 * Inside a stage, lane half h owns k in [32h, 32h+32); MFMA step s takes
 * k = 32h + 8s + [0, 8) from both operands.
 *
 * Software pipeline: the operands of step s+1 (A rows from LDS, B codes
 * dequantized in registers) are prepared while step s's 16 MFMAs run. The
 * stage barrier sits inside the last step of a stage: by then every wave
 * holds that step's operands in registers, so the barrier (a) lets the
 * freed buffer be refilled at once, keeping all NS stages in flight, and
 * (b) is followed by MFMA work that hides the latency of the next stage's
 * first LDS reads. Scales come from the per-tile table in LDS (sct: one
 * {slot 0, slot 1} pair per 128-wide k block), not from memory. */
template <int MODE, int NRB, bool EXACT, int NW, int NRBC = 0, int H0 = 0>
__device__ __forceinline__ void pf_tile(const PfTile &t, uint8_t *lds,
                                        ghip_f32x2 *sct) {
    /* NW = 4 waves (one per SIMD) or 8 (two per SIMD). Wave wv computes
     * column group cw = wv & 3 over row half hr = wv >> 2 of the tile (8
     * waves) or over all its rows (4 waves): NRBW row blocks. A stage's DMA
     * is QA + 16 one-KB loads dealt round-robin to the waves (with 8 waves
     * a 1-block tile loads its A rows twice, so every wave issues the same
     * count: identical bytes to the same LDS place). */
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    /* NRBC, H0 (8 waves, 8-block layout only): this wave computes NRBC row
     * blocks and the first row half holds H0 -- a tile of 7 blocks runs its
     * second half on 3 (no MFMAs on the empty fourth block), with loads,
     * LDS layout and barriers unchanged */
    constexpr uint32_t NRBL = NW == 8 ? (NRB >= 2 ? NRB / 2 : 1) : NRB;
    constexpr uint32_t NRBW = NRBC > 0 ? (uint32_t)NRBC : NRBL;   /* computed here */
    constexpr uint32_t HB0 = H0 > 0 ? (uint32_t)H0 : NRBL;        /* first half */
    static_assert(NRBC == 0 || (NW == 8 && NRB == 8 && NRBW <= HB0 && HB0 <= 4),
                  "short row halves: 8-wave, 8-block layout");
    constexpr uint32_t QA = NW == 8 && NRB < 2 ? 8 : 4 * NRB;
    constexpr uint32_t NA = QA / NW;              /* A loads per wave per stage */
    constexpr uint32_t NWL = 16 / NW;             /* weight loads per wave per stage */
    constexpr uint32_t LPS = NA + NWL;            /* DMA loads per wave per stage */
    /* ring depth: as many stages as the ring holds, so tiles with few rows
     * keep more weight bytes in flight (3, 4, 6, 7 stages for 8, 4, 2, 1
     * row blocks) */
    constexpr uint32_t ASTG = NRB * 32 * PF_BK * 2;
    /* WB (the full 256-row tile with 8 waves, modes 0 and 1): the weights
     * come in 128-wide k blocks (32 KB: 256 rows x one full 128-byte line
     * each, so every load instruction reads 8 whole lines instead of 16
     * half lines) through their own 2-block ring after the 3-stage A ring,
     * filling all 160 KB; the scales come by scalar loads (no table) */
    constexpr bool WB = NW == 8 && NRB == 8 && MODE < 2 && !EXACT;
    constexpr uint32_t STG = WB ? ASTG : ASTG + PF_W_STAGE;
    constexpr uint32_t NS = WB ? 3u : (PF_RING / STG < 8 ? PF_RING / STG : 8);
    constexpr uint32_t NWW = WB ? (PF_WB / 1024) / NW : 0;  /* block loads per wave */
    static_assert(NS >= 2 && LPS * (NS - 1) <= 63, "ring depth vs vmcnt range");
    static_assert(!WB || NS * ASTG + 2 * PF_WB == PF_LDS_WB, "WB layout");
    /* opaque thread id: keeps the lane-derived address math of this body
     * inside the persistent item loop instead of hoisted and held live
     * across items for every body */
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t lane = tid & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t cw = wv & 3u, hr = NW == 8 ? wv >> 2 : 0u;
    const uint32_t n = lane & 31, h = lane >> 5;
    const uint32_t K = t.K, nst = t.KS / PF_BK;

    /* the tile's scale table ({slot 0, slot 1} per 128-wide k block): this
     * thread's entry is loaded first (clamped index, unpredicated), so its
     * round trip overlaps the row-permutation loads below; it is stored
     * before the DMA prologue is issued (a wait behind the DMA would hold
     * the tile's start until the whole prologue landed) */
    const uint32_t nsc = t.KS >> 7, sb = tid < nsc ? tid : nsc - 1;
    ghip_f32x2 sv;
    if constexpr (!WB) {
        sv[0] = t.sr0[sb];
        sv[1] = t.sr1[sb];
    }

    /* --- DMA sources: a wave-uniform base (SGPRs; stage j adds j*64
     * elements) plus a 32-bit per-lane offset, so each load is one
     * SGPR-based global_load_lds with no per-load 64-bit address math ---- */
    uint32_t aofs[NA], alds[NA];
#pragma unroll
    for (int i = 0; i < (int)NA; i++) {
        const uint32_t q = wv + NW * i, qq = NW == 8 && NRB < 2 ? (q & 3u) : q;
        alds[i] = qq * 1024u;
        const uint32_t r = 8 * qq + (lane >> 3);
        const uint32_t rc = r < t.rows ? r : t.rows - 1;
        const uint32_t src = MODE == 0 ? (uint32_t)t.perm[t.row0 + rc] / t.topk
                                       : t.row0 + rc;
        const uint32_t p = (lane & 7) ^ ((r >> 1) & 7);
        aofs[i] = src * K * 2u + 16u * p;
    }
    if constexpr (!WB) {
        if (tid < nsc) sct[tid] = sv;
        for (uint32_t b = tid + NW * 64; b < nsc; b += NW * 64) {
            ghip_f32x2 v;
            v[0] = t.sr0[b];
            v[1] = t.sr1[b];
            sct[b] = v;
        }
    }
    /* WB weight block loads: instruction b of wave wv fills LDS rows 8q ..
     * 8q + 7 of the block (q = wv + 8b; 128 bytes each), rows of slot hr
     * (the same logical row order as the stage layout: row 64i + 32s + c is
     * column 32i + c of slot s's block), piece p of row r at p ^ ((r >> 1)
     * & 7); block m adds 128 m bytes */
    /* (row 8q + l/8 with q = wv + 8b is 64b + r0, r0 = 8wv + l/8 < 64: column
     * 32b + (r0 & 31), swizzle (r0 >> 1) & 7 -- load b adds 32b rows) */
    const uint8_t *wsrcB = nullptr;
    uint32_t wofsB = 0;
    if constexpr (WB) {
        wsrcB = (hr ? t.w1 : t.w0) + (size_t)(hr ? t.cb1 : t.cb0) * K;
        const uint32_t r0 = 8u * wv + (lane >> 3);
        wofsB = (r0 & 31u) * K + 16u * ((lane & 7u) ^ ((r0 >> 1) & 7u));
    }
    /* weight load i of wave wv, lane l: LDS weight row 64i + 16wv + l/4,
     * i.e. slot (wv >> 1) & 1 (uniform), column 32i + 16(wv & 1) + l/4 of
     * that slot's block, piece (l & 3) ^ ((l >> 4) & 3) */
    const uint32_t wslot = (cw >> 1) & 1u;
    const uint8_t *wbase = (wslot ? t.w1 : t.w0) + (size_t)(wslot ? t.cb1 : t.cb0) * K;
    uint32_t wofs[NWL];
#pragma unroll
    for (int b = 0; b < (int)NWL; b++) {
        const uint32_t col = 32u * ((wv + NW * b) >> 2) + 16u * (cw & 1u) + (lane >> 2);
        wofs[b] = col * K + 16u * ((lane & 3u) ^ ((lane >> 4) & 3u));
    }
    const uint8_t *abase = (const uint8_t *)t.act;
    /* part P (of 4) of stage j's loads into ring buffer b % NS: load q of
     * the stage (A rows q < NRB, weight rows NRB + i) when q % 4 == P, so a
     * stage's LPS loads spread over the four MFMA steps of the stage before
     * it instead of queueing behind each other at one point */
    auto issue_part = [&](auto part_c, uint32_t j, uint32_t b) {
        constexpr int P = decltype(part_c)::value;
        uint8_t *st = lds + (b % NS) * STG;
        const uint8_t *aj = abase + (size_t)j * PF_BK * 2;
        const uint8_t *wj = wbase + (size_t)j * PF_BK;
#pragma unroll
        for (int i = 0; i < (int)NA; i++)
            if (i % 4 == P) ghip_dma16(aj + aofs[i], st + alds[i]);
#pragma unroll
        for (int b = 0; b < (int)NWL; b++)
            if (((int)NA + b) % 4 == P)
                ghip_dma16(wj + wofs[b], st + ASTG + (wv + NW * b) * 1024);
    };
    auto issue = [&](uint32_t j, uint32_t b) {
        issue_part(std::integral_constant<int, 0>{}, j, b);
        issue_part(std::integral_constant<int, 1>{}, j, b);
        issue_part(std::integral_constant<int, 2>{}, j, b);
        issue_part(std::integral_constant<int, 3>{}, j, b);
    };
    /* WB: half P (of 2) of stage j's A loads / of weight block m's loads */
    auto issue_a = [&](auto part_c, uint32_t j) {
        constexpr int P = decltype(part_c)::value;
        uint8_t *st = lds + (j % NS) * ASTG;
        const uint8_t *aj = abase + (size_t)j * PF_BK * 2;
#pragma unroll
        for (int i = 0; i < (int)NA; i++)
            if (i % 2 == P) ghip_dma16(aj + aofs[i], st + alds[i]);
    };
    auto issue_w = [&](auto part_c, uint32_t m) {
        constexpr int P = decltype(part_c)::value;
        uint8_t *wb = lds + NS * ASTG + (m & 1u) * PF_WB;
        const uint8_t *wm = wsrcB + (size_t)m * 128u;
#pragma unroll
        for (int b = 0; b < (int)NWW; b++)
            if (b % 2 == P)
                ghip_dma16(wm + (size_t)(32u * b) * K + wofsB, wb + (wv + NW * b) * 1024);
    };

    /* --- operand read offsets inside a stage --------------------------- */
    /* slot 1's rows follow slot 0's 32 rows later in both layouts (the
     * swizzle depends on n only): one offset register per u, the slot-1
     * read at a constant distance BD */
    constexpr uint32_t BD = WB ? 32u * 128u : 32u * 64u;
    uint32_t aoff[4], boff0[2];
#pragma unroll
    for (int s = 0; s < 4; s++)
        aoff[s] = n * 128 + 16 * (((4 * h) | s) ^ ((n >> 1) & 7));
#pragma unroll
    for (int u = 0; u < 2; u++) {
        if constexpr (WB) {
            /* in the weight block, from its base; an odd stage reads the
             * other 64 bytes of each line: offset ^ 64 (piece ^ 4) */
            const uint32_t ph = ((2 * h + u) ^ ((n >> 1) & 7)) * 16;
            boff0[u] = (64 * cw + n) * 128 + ph;
        } else {
            const uint32_t ph = ((2 * h + u) ^ ((n >> 2) & 3)) * 16;
            boff0[u] = ASTG + (64 * cw + n) * 64 + ph;
        }
    }
    /* B codes of stage j: WB reads weight block j / 2, else the stage */
    auto bsrc = [&](uint32_t j) -> const uint8_t * {
        if constexpr (WB) return lds + NS * ASTG + ((j >> 1) & 1u) * PF_WB;
        else return lds + (j % NS) * STG;
    };
    auto bpar = [&](uint32_t j) -> uint32_t { return WB ? (j & 1u) * 64u : 0u; };

    ghip_f32x16 a0[NRBW], a1[NRBW];
    /* this wave's first row block in the stage's A rows */
    const uint32_t arow0 = NW == 8 && NRB >= 2 ? hr * HB0 * 32u * 128u : 0u;
#pragma unroll
    for (int rb = 0; rb < (int)NRBW; rb++)
#pragma unroll
        for (int i = 0; i < 16; i++) { a0[rb][i] = 0.0f; a1[rb][i] = 0.0f; }

    /* prologue: up to NS - 1 stages in flight, then stage 0's step-0
     * operands; stage j's steps load stage j + NS - 1 (while it exists)
     * into the buffer freed by stage j - 1. No load is issued past the
     * tile's last stage, so none is left in flight when the tile ends: the
     * next item (possibly another body with another LDS layout) starts on
     * a quiet ring. */
    ghip_f32x2 sc, scn;                          /* WB: scales of this / the next k block */
    if constexpr (WB) {
        /* weight block 0 first, then A stages 0 and 1 (nst >= 2): waiting
         * for stage 0's A loads covers block 0 */
        issue_w(std::integral_constant<int, 0>{}, 0u);
        issue_w(std::integral_constant<int, 1>{}, 0u);
        issue_a(std::integral_constant<int, 0>{}, 0u);
        issue_a(std::integral_constant<int, 1>{}, 0u);
        issue_a(std::integral_constant<int, 0>{}, 1u);
        issue_a(std::integral_constant<int, 1>{}, 1u);
        sc[0] = ghip_sload(t.sr0, 0);
        sc[1] = ghip_sload(t.sr1, 0);
        const uint32_t b1i = nst > 2 ? 1u : 0u;
        scn[0] = ghip_sload(t.sr0, b1i);
        scn[1] = ghip_sload(t.sr1, b1i);
        GHIP_VMCNT(NA);
    } else {
#pragma unroll
        for (uint32_t i = 0; i + 1 < NS; i++)
            if (i < nst) issue(i, i);
        ghip_wait_stages<LPS, NS - 2>(nst - 1);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);          /* lgkmcnt(0): scale table */
    __builtin_amdgcn_s_barrier();
    ghip_u32x4 q0[2], q1[2];
    ghip_bf16x8 av[NRBW], an[NRBW], b0, b1, nb0, nb1;
    {
        const uint8_t *st = lds;
        const uint8_t *sb0 = bsrc(0);
        if constexpr (!WB) sc = sct[0];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            q0[u] = *(const ghip_u32x4 *)(sb0 + boff0[u]);
            q1[u] = *(const ghip_u32x4 *)(sb0 + boff0[u] + BD);
        }
#pragma unroll
        for (int rb = 0; rb < (int)NRBW; rb++)
            av[rb] = *(const ghip_bf16x8 *)(st + arow0 + rb * 32 * 128 + aoff[0]);
        b0 = pf_deq8<EXACT>(q0[0][0], q0[0][1], sc[0]);
        b1 = pf_deq8<EXACT>(q1[0][0], q1[0][1], sc[1]);
    }

    /* one stage; NEXT: stage j+1 exists (its barrier, the refill of the
     * freed buffer and its step-0 reads run in step 3); REFILL: stage
     * j + NS - 1 exists and is loaded during this one. Branch-free inside,
     * so each step is one scheduling region in which the next operands' LDS
     * reads and dequant interleave with the MFMAs. */
    auto stage = [&](uint32_t j, auto next_c, auto refill_c, auto par_c) {
        constexpr bool NEXT = decltype(next_c)::value;
        constexpr bool REFILL = decltype(refill_c)::value;
        constexpr int PAR = decltype(par_c)::value;       /* WB: j % 2 */
        const uint8_t *st = lds + (j % NS) * STG;
        const uint32_t ld = j + NS - 1;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            if constexpr (WB) {
                /* an even stage issues weight block j/2 + 1 (steps 0, 1)
                 * ahead of stage j + 2's A rows (steps 2, 3), so waiting for
                 * those A rows covers the block too */
                if (REFILL && PAR == 0 && s == 0) issue_w(std::integral_constant<int, 0>{}, (j >> 1) + 1u);
                if (REFILL && PAR == 0 && s == 1) issue_w(std::integral_constant<int, 1>{}, (j >> 1) + 1u);
                if (REFILL && s == 2) issue_a(std::integral_constant<int, 0>{}, j + 2u);
                if (REFILL && s == 3) issue_a(std::integral_constant<int, 1>{}, j + 2u);
            } else {
                if (REFILL && s == 0) issue_part(std::integral_constant<int, 0>{}, ld, ld);
                if (REFILL && s == 1) issue_part(std::integral_constant<int, 1>{}, ld, ld);
                if (REFILL && s == 2) issue_part(std::integral_constant<int, 2>{}, ld, ld);
                if (REFILL && s == 3) issue_part(std::integral_constant<int, 3>{}, ld, ld);
            }
            if (s < 3) {
                /* step s+1 of this stage: A rows from LDS, B codes already
                 * in registers */
                const int u = (s + 1) >> 1, v = 2 * ((s + 1) & 1);
#pragma unroll
                for (int rb = 0; rb < (int)NRBW; rb++)
                    an[rb] = *(const ghip_bf16x8 *)(st + arow0 + rb * 32 * 128 + aoff[s + 1]);
                nb0 = pf_deq8<EXACT>(q0[u][v], q0[u][v + 1], sc[0]);
                nb1 = pf_deq8<EXACT>(q1[u][v], q1[u][v + 1], sc[1]);
            } else if (NEXT) {
                /* stage barrier: own DMA for stage j+1 done (later stages
                 * may stay in flight), own reads of stage j done; then a
                 * bare barrier (no fence: a fence would drain the DMA
                 * ring) after which buffer j % NS is free for stage j+NS.
                 * Stages up to min(j + NS - 1, nst - 1) are issued by now,
                 * in order: min(NS - 2, nst - 2 - j) of them after j+1 */
                if constexpr (WB) {
                    if (!REFILL) GHIP_VMCNT(0);
                    else if (PAR == 0) GHIP_VMCNT(NA + NWW);
                    else GHIP_VMCNT(NA);
                } else {
                    if (REFILL) GHIP_VMCNT(LPS * (NS - 2));
                    else ghip_wait_stages<LPS, NS - 2>(nst - 2 - j);
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                const uint8_t *sn = lds + ((j + 1) % NS) * STG;
                const uint8_t *sbn = bsrc(j + 1);
                const uint32_t bx = bpar(j + 1);
                if constexpr (WB) {
                    if (PAR == 1) {                       /* stage j + 1 opens k block (j+1)/2 */
                        sc = scn;
                        const uint32_t mb = ((j + 1) >> 1) + 1u;
                        if (mb < (nst >> 1)) {
                            scn[0] = ghip_sload(t.sr0, mb);
                            scn[1] = ghip_sload(t.sr1, mb);
                        }
                    }
                } else {
                    sc = sct[(j + 1) >> 1];
                }
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    q0[u] = *(const ghip_u32x4 *)(sbn + (boff0[u] ^ bx));
                    q1[u] = *(const ghip_u32x4 *)(sbn + (boff0[u] ^ bx) + BD);
                }
#pragma unroll
                for (int rb = 0; rb < (int)NRBW; rb++)
                    an[rb] = *(const ghip_bf16x8 *)(sn + arow0 + rb * 32 * 128 + aoff[0]);
                nb0 = pf_deq8<EXACT>(q0[0][0], q0[0][1], sc[0]);
                nb1 = pf_deq8<EXACT>(q1[0][0], q1[0][1], sc[1]);
            }
#pragma unroll
            for (int rb = 0; rb < (int)NRBW; rb++) {
                a0[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[rb], b0, a0[rb], 0, 0, 0);
                a1[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[rb], b1, a1[rb], 0, 0, 0);
            }
            /* interleave the next step's LDS reads and dequant (and, at a
             * stage boundary, the DMA refill) between this step's MFMAs */
            if (s == 3 && NEXT) {
                /* 5 + NRB LDS reads (scales, B codes, A rows), then the
                 * dequant of the next step's B */
#pragma unroll
                for (int i = 0; i < 2 * (int)NRBW; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   /* MFMA */
                    if (i < 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0); /* DS read */
                    if (i == 2) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (i >= 3 && i < 3 + (int)NRBW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (i >= (NW == 8 ? 3 : 5)) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0); /* VALU */
                }
            } else if (s < 3) {
#pragma unroll
                for (int i = 0; i < 2 * (int)NRBW; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (i < (int)NRBW) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, NW == 8 ? 4 : 2, 0);
                }
            }
            /* step boundary: a scheduling region per step, so the next
             * step's reads stay between this step's MFMAs instead of being
             * pulled down next to their consumers */
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int rb = 0; rb < (int)NRBW; rb++) av[rb] = an[rb];
            b0 = nb0;
            b1 = nb1;
        }
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    if constexpr (WB) {
        /* stage pairs (nst is even: K % 128 == 0) */
        uint32_t j = 0;
        for (; j + 2 < nst; j += 2) {
            stage(j, std::true_type{}, std::true_type{}, P0{});
            stage(j + 1, std::true_type{}, std::true_type{}, P1{});
        }
        stage(nst - 2, std::true_type{}, std::false_type{}, P0{});
        stage(nst - 1, std::false_type{}, std::false_type{}, P1{});
    } else {
        uint32_t j = 0;
        for (; j + NS - 1 < nst; j++) stage(j, std::true_type{}, std::true_type{}, P0{});
        for (; j + 1 < nst; j++) stage(j, std::true_type{}, std::false_type{}, P0{});
        stage(nst - 1, std::false_type{}, std::false_type{}, P0{});
    }

    /* epilogue: lane (n, h), register i of row block rb holds output row
     * rowbase + rb*32 + 8*(i/4) + 4*h + i%4, column n of each slot */
    const uint32_t rowbase = hr * HB0 * 32;
    if constexpr (MODE == 2) {
        const uint32_t c0 = t.cb0 + 32 * cw + n, c1 = t.cb1 + 32 * cw + n;
#pragma unroll
        for (int rb = 0; rb < (int)NRBW; rb++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t r = rowbase + rb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
                if (r < t.rows) {
                    float *of = t.outf + (size_t)(t.row0 + r) * t.N;
                    of[c0] = a0[rb][i];
                    of[c1] = a1[rb][i];
                }
            }
        }
    } else {
        /* Staged through a wave-private LDS area so the stores are
         * row-contiguous 16-byte vectors: every wave's reads of the ring
         * are done first (the area overlaps the ring). MODE 0 stages the
         * wave's 32 h columns (64 B per row), MODE 1 its two 32-column
         * groups c0 | c1 (128 B per row). A row r sits at r ^ ((r >> 2) & 1)
         * (MODE 0) or its two 64-byte halves swap when (r >> 2) & 1
         * (MODE 1), so lanes h = 0 and 1 (rows r and r + 4) write to
         * different banks. */
        /* RW: rows this wave computed; areas are HB0 * 32 rows apart */
        constexpr uint32_t RW = NRBW * 32, RB = MODE == 0 ? 64 : 128;
        __builtin_amdgcn_s_waitcnt(0xc07f);            /* lgkmcnt(0) */
        __builtin_amdgcn_s_barrier();
        uint8_t *sw = lds + wv * (HB0 * 32u * RB);
#pragma unroll
        for (int rb = 0; rb < (int)NRBW; rb++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t r = rb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
                if (MODE == 0) {
                    const uint32_t pr = r ^ ((r >> 2) & 1u);
                    *(uint16_t *)(sw + pr * 64u + n * 2u) = pf_swiglu(a0[rb][i], a1[rb][i], t.limit);
                } else {
                    const uint32_t x = ((r >> 2) & 1u) * 64u;
                    *(uint16_t *)(sw + r * 128u + ((n * 2u) ^ x)) = pf_bf16_bits(a0[rb][i]);
                    *(uint16_t *)(sw + r * 128u + ((64u + n * 2u) ^ x)) = pf_bf16_bits(a1[rb][i]);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);            /* the wave's own LDS writes */
        __builtin_amdgcn_wave_barrier();
        const uint32_t p = lane & 3u;
        if (MODE == 0) {
            /* lane: row lane/4 + 16j, 16 bytes at column 8p of the wave's 32 */
            uint16_t *ob = t.out + (size_t)(t.row0 + rowbase) * t.N + t.cb0 + 32 * cw + 8 * p;
#pragma unroll
            for (int j = 0; j < (int)RW / 16; j++) {
                const uint32_t rr = (lane >> 2) + 16u * j, prr = rr ^ ((rr >> 2) & 1u);
                const ghip_u32x4 v = *(const ghip_u32x4 *)(sw + prr * 64u + p * 16u);
                if (rowbase + rr < t.rows) *(ghip_u32x4 *)(ob + (size_t)rr * t.N) = v;
            }
        } else {
            /* lane: row lane/8 + 8j, group (lane/4) & 1, 16 bytes at column 8p */
            const uint32_t gs = (lane >> 2) & 1u;
            uint16_t *ob = t.out + (size_t)(t.row0 + rowbase) * t.N + (gs ? t.cb1 : t.cb0)
                         + 32 * cw + 8 * p;
#pragma unroll
            for (int j = 0; j < (int)RW / 8; j++) {
                const uint32_t rr = (lane >> 3) + 8u * j, x = ((rr >> 2) & 1u) * 64u;
                const ghip_u32x4 v = *(const ghip_u32x4 *)(sw + rr * 128u + ((gs * 64u + p * 16u) ^ x));
                if (rowbase + rr < t.rows) *(ghip_u32x4 *)(ob + (size_t)rr * t.N) = v;
            }
        }
    }
}

/* MODE 0: act = x [T, dim], rows gathered by token (perm[s] / topk);
 *         out = H [P, inter] (sorted rows), SwiGLU epilogue.
 * MODE 1: act = H [P, inter] (sorted rows); out = O [P, dim] (sorted rows),
 *         bf16 expert outputs.
 * Grid: G (multiple of 8) workgroups of NW * 64 threads, one per CU. The
 * body is chosen once per tile: 8, 4, 2 or 1 row blocks (the smallest that
 * holds the tile), or the exact-decode body for an expert with NaN codes.
 *
 * Items (tile, column block) are grouped by XCD: XCD x owns tiles x, x + 8,
 * ... and its workgroups share each tile's column blocks, so a tile's
 * gathered activation rows are read into one L2. With NW = 8 (routings
 * that fill tiles: items of one size) an XCD's workgroups take its items
 * round-robin. With NW = 4 (sparse routings: tiles of 1 to 256 rows, items
 * of very different cost) they take them from the XCD's queue, a counter
 * in hdr that every grab bumps, and, once it is empty, from the other XCDs'
 * queues in turn: no workgroup idles while another still holds a backlog.
 * A grab past a queue's end moves on to the next queue, so every workgroup
 * leaves the loop after at most one failed grab per queue. */
template <int MODE, int NW>
__global__ __launch_bounds__(NW * 64, 1) void k_pf_gemm(
    GhipBank bank, const uint16_t *__restrict__ act,
    const int32_t *__restrict__ perm, const uint4 *__restrict__ tiles,
    uint32_t *__restrict__ hdr, uint32_t nblk, uint32_t topk,
    float limit, uint16_t *__restrict__ out) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t pf_lds[];
    /* persistent: one workgroup per CU; workgroup b runs on XCD b % 8 and
     * that XCD takes tiles x, x+8, ...; its workgroups share each tile's
     * column blocks (same activation rows, one L2) */
    __shared__ uint32_t s_item;
    const uint32_t ntiles = hdr[PF_HDR_NTILES];
    const uint32_t x = blockIdx.x & 7u, c = blockIdx.x >> 3, per = gridDim.x >> 3;
    const uint32_t ntx = ntiles > x ? (ntiles - x + 7) >> 3 : 0;
    const uint32_t items = ntx * nblk;
    const uint32_t K = MODE == 0 ? bank.dim : bank.inter;
    const uint32_t nkb = K >> 7;
    constexpr bool DYN = NW == 4;
    constexpr uint32_t NONE = 0xffffffffu;
    /* dynamic items: thread 0 grabs (queue y, index i) and publishes the
     * tile index * nblk + column block in s_item (NONE when every queue is
     * empty); yq = queues found empty so far (thread 0 only) */
    uint32_t *qc = hdr + PF_HDR_Q + 8u * MODE;
    uint32_t yq = 0;
    auto grab = [&]() -> uint32_t {
        while (yq < 8u) {
            const uint32_t y = (x + yq) & 7u;
            const uint32_t ny = ntiles > y ? (ntiles - y + 7) >> 3 : 0;
            const uint32_t i = __hip_atomic_fetch_add(qc + y, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            if (i < ny * nblk) return (y + 8u * (i / nblk)) * nblk + i % nblk;
            yq++;
        }
        return NONE;
    };
    if constexpr (DYN) {
        if (threadIdx.x == 0) s_item = grab();
        __syncthreads();
    }
    /* static items: the next item's tile record is loaded while this item
     * runs */
    uint4 tdn = make_uint4(0u, 0u, 0u, 0u);
    if (!DYN && c < items) tdn = tiles[x + 8 * (c / nblk)];
    for (uint32_t k = c;; k += per) {
        uint32_t nb;
        uint4 td;
        if constexpr (DYN) {
            const uint32_t it = __builtin_amdgcn_readfirstlane(s_item);
            if (it == NONE) break;
            nb = it % nblk;
            td = tiles[it / nblk];
        } else {
            if (k >= items) break;
            nb = k % nblk;
            td = tdn;
            if (k + per < items) tdn = tiles[x + 8 * ((k + per) / nblk)];
        }
        const uint32_t e = td.x;
        PfTile t;
        t.act = act;
        t.perm = perm;
        t.out = out;
        t.row0 = td.y;
        t.rows = td.z;
        t.topk = topk;
        t.limit = limit;
        t.K = K;
        t.KS = K;
        t.outf = nullptr;
        t.N = MODE == 0 ? bank.inter : bank.dim;
        const uint8_t *slab = bank.base + (size_t)e * bank.stride;
        if (MODE == 0) {
            t.cb0 = t.cb1 = nb * 128;
            t.w0 = slab + bank.off_gw;
            t.w1 = slab + bank.off_uw;
            t.sr0 = (const float *)(slab + bank.off_gs) + (size_t)nb * nkb;
            t.sr1 = (const float *)(slab + bank.off_us) + (size_t)nb * nkb;
        } else {
            t.cb0 = nb * 256;
            t.cb1 = nb * 256 + 128;
            t.w0 = t.w1 = slab + bank.off_dw;
            t.sr0 = (const float *)(slab + bank.off_ds) + (size_t)(2 * nb) * nkb;
            t.sr1 = (const float *)(slab + bank.off_ds) + (size_t)(2 * nb + 1) * nkb;
        }
        /* the tile's scale table is filled by the body and made visible by
         * its prologue barrier (the previous item's trailing barrier ordered
         * all reads of the old table); td.w = the expert's NaN-code flag */
        ghip_f32x2 *sct = (ghip_f32x2 *)(pf_lds + PF_RING);
        const uint32_t nrb = (t.rows + 31) >> 5;
        if (td.w) pf_tile<MODE, PF_RB, true, NW>(t, pf_lds, sct);
        else if (NW == 8 && nrb == 7) {
            /* 7 blocks: the second row half computes 3 (same loads) */
            if constexpr (NW == 8) {
                if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 2)
                    pf_tile<MODE, 8, false, NW, 3, 4>(t, pf_lds, sct);
                else
                    pf_tile<MODE, 8, false, NW, 4, 4>(t, pf_lds, sct);
            }
        }
        else if (nrb > 4) pf_tile<MODE, 8, false, NW>(t, pf_lds, sct);
        else if (nrb > 2) pf_tile<MODE, 4, false, NW>(t, pf_lds, sct);
        else if (nrb > 1) pf_tile<MODE, 2, false, NW>(t, pf_lds, sct);
        else              pf_tile<MODE, 1, false, NW>(t, pf_lds, sct);
        if constexpr (DYN) {
            /* every wave has read s_item (the body holds barriers) */
            if (threadIdx.x == 0) s_item = grab();
            __builtin_amdgcn_s_waitcnt(0xc07f);  /* lgkmcnt(0): s_item written */
        }
        /* every wave is done with the LDS ring before the next item's
         * prologue refills it (and, dynamic, s_item is published) */
        __builtin_amdgcn_s_barrier();
    }
    /* each tile body waits for every load it issued (none past its last
     * stage), so nothing is in flight here; kept as a guard before the
     * workgroup's LDS is released */
    GHIP_VMCNT(0);
}

/* ------------------------------------------------------------------------ */
/* dense FP8-block GEMM (the fp8blk_linear hook at M > the GEMV range)      */
/* ------------------------------------------------------------------------ */

/* Y [M, N] = bf16(X [M, K] . dequant(W [N, K])^T), the composition of
 * c/gdsa.h:525-534 (dequant_mt then gemm_mt) without the BF16 weight copy:
 * the tile body above on tiles of bm rows of X (256, 128, 64 or 32, chosen
 * by the launcher) x 256 rows of W (two 128-row scale blocks).
 *
 * With S > 1 the K range is split too (split-K for launches with fewer
 * tiles than CUs): split s covers k blocks [s*nkb/S, (s+1)*nkb/S) and
 * writes its fp32 partial sums to part[s] [M, N] (MODE 2); k_splitk_sum
 * then adds the S partials in ascending s and rounds once. With S == 1 the
 * tile writes bf16 Y directly (MODE 1).
 *
 * Items ((row tile, split) unit, column block) are dealt to the 8 XCDs
 * (workgroup b runs on XCD b % 8) as an R x (8/R) grid: XCD x owns the
 * units u == x / (8/R) (mod R) and the column blocks nb == x % (8/R)
 * (mod 8/R), so each XCD's L2 holds 1/R of X's rows and (R/8) of the
 * weights; the launcher picks R to minimize the bytes fetched into the
 * L2s, (8/R) |X| + R |W|. exact_dev: NULL or a device flag, nonzero when W
 * holds a NaN code (0x7F/0xFF) and the exact integer decode must be
 * used. */
__global__ __launch_bounds__(256, 1) void k_fp8_gemm(
    const uint8_t *__restrict__ codes, const float *__restrict__ scales,
    const uint16_t *__restrict__ x, uint16_t *__restrict__ y, float *__restrict__ part,
    uint32_t M, uint32_t N, uint32_t K, uint32_t bm, uint32_t S, uint32_t R,
    const uint32_t *__restrict__ exact_dev) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t pf_lds[];
    const uint32_t nkb = K >> 7, nblk = N >> 8, tiles = (M + bm - 1) / bm;
    const uint32_t rows_u = tiles * S;             /* (row tile, split) units */
    const bool exact = exact_dev && *exact_dev;
    const uint32_t xcd = blockIdx.x & 7u, c = blockIdx.x >> 3, per = gridDim.x >> 3;
    const uint32_t C = 8u / R, xr = xcd / C, xc = xcd - xr * C;
    const uint32_t nru = rows_u > xr ? (rows_u - xr + R - 1) / R : 0;
    const uint32_t nnb = nblk > xc ? (nblk - xc + C - 1) / C : 0;
    for (uint32_t q = c; q < nru * nnb; q += per) {
        const uint32_t ru = xr + R * (q / nnb), nb = xc + C * (q % nnb);
        const uint32_t tile = ru / S, sp = ru - tile * S;
        const uint32_t kb0 = sp * nkb / S, kb1 = (sp + 1) * nkb / S;
        PfTile t;
        t.act = x + (size_t)kb0 * 128;
        t.perm = nullptr;
        t.out = y;
        t.outf = part + (size_t)sp * M * N;
        t.row0 = tile * bm;
        t.rows = M - t.row0 < bm ? M - t.row0 : bm;
        t.topk = 1;
        t.limit = 0.0f;
        t.K = K;
        t.KS = (kb1 - kb0) * 128;
        t.N = N;
        t.cb0 = nb * 256;
        t.cb1 = nb * 256 + 128;
        t.w0 = t.w1 = codes + (size_t)kb0 * 128;
        t.sr0 = scales + (size_t)(2 * nb) * nkb + kb0;
        t.sr1 = scales + (size_t)(2 * nb + 1) * nkb + kb0;
        ghip_f32x2 *sct = (ghip_f32x2 *)(pf_lds + PF_RING);
        const uint32_t nrb = (t.rows + 31) >> 5;
        if (S > 1) {
            if (exact) pf_tile<2, PF_RB, true, 4>(t, pf_lds, sct);
            else if (nrb > 4) pf_tile<2, 8, false, 4>(t, pf_lds, sct);
            else if (nrb > 2) pf_tile<2, 4, false, 4>(t, pf_lds, sct);
            else if (nrb > 1) pf_tile<2, 2, false, 4>(t, pf_lds, sct);
            else              pf_tile<2, 1, false, 4>(t, pf_lds, sct);
        } else {
            if (exact) pf_tile<1, PF_RB, true, 4>(t, pf_lds, sct);
            else if (nrb > 4) pf_tile<1, 8, false, 4>(t, pf_lds, sct);
            else if (nrb > 2) pf_tile<1, 4, false, 4>(t, pf_lds, sct);
            else if (nrb > 1) pf_tile<1, 2, false, 4>(t, pf_lds, sct);
            else              pf_tile<1, 1, false, 4>(t, pf_lds, sct);
        }
        __builtin_amdgcn_s_barrier();
    }
    GHIP_VMCNT(0);
}

/* y = bf16(part[0] + part[1] + ... + part[S-1]) elementwise, ascending s
 * (a fixed order: deterministic); 4 outputs per thread. */
__global__ __launch_bounds__(256) void k_splitk_sum(const float *__restrict__ part,
                                                    uint32_t S, size_t n,
                                                    uint16_t *__restrict__ y) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    ghip_f32x4 a = *(const ghip_f32x4 *)(part + i);
    for (uint32_t sp = 1; sp < S; sp++) {
        const ghip_f32x4 b = *(const ghip_f32x4 *)(part + (size_t)sp * n + i);
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = a[j] + b[j];
    }
    /* 16-bit stores: y needs only its element alignment */
#pragma unroll
    for (int j = 0; j < 4; j++) y[i + j] = (uint16_t)ghip_bf16_bits(a[j]);
}

/* ------------------------------------------------------------------------ */
/* ordered combine                                                          */
/* ------------------------------------------------------------------------ */

/* Workgroup (t, c) combines columns [2048c, 2048c + 2048) of token t, 8
 * per thread: the token's kept pairs in ascending expert id,
 * contrib = bf16(bf16(o) * w), y = bf16(y + contrib), y from +0
 * (c/gmoe.h:307-320). One wave orders the token's pairs once into LDS
 * (instead of every thread re-reading and re-sorting them); then each
 * thread loads its rows of O in batches of 8 and adds them in that order. */
__global__ __launch_bounds__(256) void k_pf_combine(
    const uint16_t *__restrict__ O, const int32_t *__restrict__ pos,
    const int32_t *__restrict__ idx, const float *__restrict__ w, uint32_t T,
    uint32_t topk, uint32_t topk_p, uint32_t dim, uint16_t *__restrict__ out) {
    __shared__ int32_t srow[PF_MAXK];
    __shared__ float sw[PF_MAXK];
    __shared__ uint32_t sn;
    __shared__ int32_t sshared;
    const uint32_t cpt = (dim + 2047) / 2048;          /* workgroups per token */
    const uint32_t t = blockIdx.x / cpt, c = blockIdx.x - t * cpt;
    const uint32_t tid = threadIdx.x;
    if (tid < 64) {
        /* lane j holds routed pair j; a kept pair's rank among the kept
         * pairs by expert id is its slot in the ordered list (ids of kept
         * pairs are distinct: repeats were dropped by the permutation). The
         * shared expert's pair (slot topk, when topk_p > topk) is added
         * after them. */
        const uint32_t j = tid;
        const size_t p = (size_t)t * topk + j;
        const int32_t s = j < topk ? pos[(size_t)t * topk_p + j] : -1;
        const int32_t e = s >= 0 ? idx[p] : 0x7fffffff;
        const float wj = j < topk ? w[p] : 0.0f;
        if (tid == 0)
            sshared = topk_p > topk ? pos[(size_t)t * topk_p + topk] : -1;
        uint32_t rank = 0;
        for (uint32_t q = 0; q < topk; q++) {
            const int32_t eq = __shfl(e, (int)q, 64);
            rank += eq < e;
        }
        const uint64_t kept = __ballot(s >= 0);
        if (s >= 0) {
            srow[rank] = s;
            sw[rank] = wj;
        }
        if (tid == 0) sn = (uint32_t)__popcll(kept);
    }
    __syncthreads();
    const uint32_t d = c * 2048 + tid * 8;
    if (t >= T || d >= dim) return;
    const uint32_t n = sn;
    float y[8];
#pragma unroll
    for (int q = 0; q < 8; q++) y[q] = 0.0f;
    for (uint32_t r0 = 0; r0 < n; r0 += 8) {
        /* the rows and weights of up to 8 pairs first (one LDS wait), then
         * all their loads (rows past n re-read the last one, unused) */
        int32_t rr[8];
        float wr[8];
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const uint32_t i = min(r0 + (uint32_t)r, n - 1u);
            rr[r] = srow[i];
            wr[r] = sw[i];
        }
        ghip_u32x4 v[8];
#pragma unroll
        for (int r = 0; r < 8; r++) v[r] = *(const ghip_u32x4 *)(O + (size_t)rr[r] * dim + d);
        /* an unconditional use of each row pins its load here, so all are
         * in flight at once (the compiler would otherwise sink each load
         * behind the exit test before its row's arithmetic) */
#pragma unroll
        for (int r = 0; r < 8; r++) asm volatile("" ::"v"(v[r]));
#pragma unroll
        for (int r = 0; r < 8; r++) {
            if (r0 + r >= n) break;
#pragma unroll
            for (int q = 0; q < 8; q += 2) {
                /* two elements a step: bf16 -> f32, the weight, the RNE
                 * narrows of the product and of the sum on the packed
                 * hardware convert (the reference's bits for every finite
                 * value, c/gmoe.h:307-320) */
                const uint32_t pr = v[r][q >> 1];
                float2 c = pf_bf16_round2(__uint_as_float(pr << 16) * wr[r],
                                          __uint_as_float(pr & 0xffff0000u) * wr[r]);
                float2 s2 = pf_bf16_round2(y[q] + c.x, y[q + 1] + c.y);
                y[q] = s2.x;
                y[q + 1] = s2.y;
            }
        }
    }
    const int32_t ss = sshared;
    if (ss >= 0) {
        /* the shared expert, last, one more rounding: out = bf16(y + sh) */
        const ghip_u32x4 v = *(const ghip_u32x4 *)(O + (size_t)ss * dim + d);
#pragma unroll
        for (int q = 0; q < 8; q++)
            y[q] = y[q] + ghip_bf16_f32((v[q >> 1] >> (16 * (q & 1))) & 0xffffu);
    }
    ghip_u32x4 r;
#pragma unroll
    for (int q = 0; q < 4; q++)
        r[q] = ghip_bf16_bits(y[2 * q]) | (ghip_bf16_bits(y[2 * q + 1]) << 16);
    *(ghip_u32x4 *)(out + (size_t)t * dim + d) = r;
}

/* ------------------------------------------------------------------------ */

extern "C" size_t ghip_moe_prefill_max_tiles(size_t pairs, uint32_t n_experts) {
    return (pairs + PF_BM - 1) / PF_BM + n_experts;
}

extern "C" size_t ghip_moe_prefill_chunks(size_t pairs) {
    return (pairs + PF_CHUNK - 1) / PF_CHUNK;
}

extern "C" hipError_t ghip_launch_moe_prefill(const GhipBank *bank,
                                              const uint16_t *x, size_t T,
                                              const int32_t *idx, const float *w,
                                              int topk, float limit, uint16_t *out,
                                              const GhipMoePrefillWs *ws,
                                              const hipEvent_t *ev,
                                              hipStream_t st) {
    if (!bank || !ws || !x || !idx || !w || !out) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const uint32_t dim = bank->dim, inter = bank->inter, E = bank->n_experts;
    /* with a shared expert every token has one more pair (the shared
     * expert, id E, slot topk): Ep experts, topk_p slots per token */
    const uint32_t sh = bank->has_shared ? 1u : 0u, Ep = E + sh;
    const uint32_t topk_p = (uint32_t)topk + sh;
    if (topk <= 0 || topk > PF_MAXK || E == 0 || Ep > PF_MAXE)
        return hipErrorInvalidValue;
    if (dim == 0 || inter == 0 || dim % 256 || inter % 128) return hipErrorInvalidValue;
    if (dim / 128 > PF_SCT_MAX || inter / 128 > PF_SCT_MAX) return hipErrorInvalidValue;
    const size_t P = T * (size_t)topk_p;
    if (P > ws->cap_pairs || P > 0x7fffffffu) return hipErrorInvalidValue;
    if (ws->n_cu == 0 || ws->n_cu % 8) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)bank->base & 15)
        || (bank->stride & 15) || (bank->off_gw & 15) || (bank->off_uw & 15)
        || (bank->off_dw & 15) || (bank->off_gs & 3) || (bank->off_us & 3)
        || (bank->off_ds & 3))
        return hipErrorInvalidValue;
    const uint32_t nch = (uint32_t)ghip_moe_prefill_chunks(P);
    const size_t mt = ghip_moe_prefill_max_tiles(P, Ep);
    hipEvent_t e0 = ev ? ev[0] : nullptr, e1 = ev ? ev[1] : nullptr;
    hipEvent_t e2 = ev ? ev[2] : nullptr, e3 = ev ? ev[3] : nullptr;
    hipEvent_t e4 = ev ? ev[4] : nullptr, e5 = ev ? ev[5] : nullptr;
    hipEvent_t e6 = ev ? ev[6] : nullptr, e7 = ev ? ev[7] : nullptr;
    hipError_t e;
    if ((e = ghip_launch_fill_u32(ws->hdr, PF_HDR_WORDS, 0u, st)) != hipSuccess) return e;
    GHIP_LAUNCH(e0, nullptr, k_pf_count, dim3(nch), dim3(1024), Ep * 4, st, idx,
                (uint32_t)P, (uint32_t)topk, topk_p, E, ws->cnt, ws->eid, ws->hdr,
                bank->err);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_pf_scan, dim3(1), dim3(1024), 0, st, ws->cnt, nch, Ep,
                       bank->nan_flags, (uint4 *)ws->tiles, ws->hdr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GHIP_LAUNCH(nullptr, e1, k_pf_scatter, dim3(nch), dim3(1024), 16 * Ep * 4, st,
                ws->eid, (uint32_t)P, Ep, ws->cnt, ws->perm, ws->pos);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t lds = PF_LDS, lds8 = PF_LDS_WB;
    (void)mt;
    const uint32_t g0 = ws->n_cu, g1 = ws->n_cu;
    /* two waves per SIMD when the tiles are mostly full (on average at
     * least half a 256-row tile per expert): one wave's MFMAs cover the
     * other's DMA issue; sparse routings (mostly short tiles) keep one wave
     * per SIMD, which wastes no MFMAs on a half-empty row split */
    const bool full = P >= (size_t)Ep * (PF_BM / 2);
    if (full)
        GHIP_LAUNCH(e2, e3, (k_pf_gemm<0, 8>), dim3(g0), dim3(512), lds8, st, *bank,
                    x, ws->perm, (const uint4 *)ws->tiles, ws->hdr, inter / 128,
                    topk_p, limit, ws->h);
    else
        GHIP_LAUNCH(e2, e3, (k_pf_gemm<0, 4>), dim3(g0), dim3(256), lds, st, *bank,
                    x, ws->perm, (const uint4 *)ws->tiles, ws->hdr, inter / 128,
                    topk_p, limit, ws->h);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (full)
        GHIP_LAUNCH(e4, e5, (k_pf_gemm<1, 8>), dim3(g1), dim3(512), lds8, st, *bank,
                    ws->h, ws->perm, (const uint4 *)ws->tiles, ws->hdr, dim / 256,
                    topk_p, limit, ws->o);
    else
        GHIP_LAUNCH(e4, e5, (k_pf_gemm<1, 4>), dim3(g1), dim3(256), lds, st, *bank,
                    ws->h, ws->perm, (const uint4 *)ws->tiles, ws->hdr, dim / 256,
                    topk_p, limit, ws->o);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t nblk_c = T * (size_t)((dim + 2047) / 2048);
    GHIP_LAUNCH(e6, e7, k_pf_combine, dim3((uint32_t)nblk_c), dim3(256),
                0, st, ws->o, ws->pos, idx, w, (uint32_t)T, (uint32_t)topk, topk_p, dim,
                out);
    return hipGetLastError();
}

extern "C" int ghip_fp8_gemm_fits(size_t M, size_t N, size_t K, const void *codes,
                                  const void *x, const void *y) {
    return M > 0 && M <= 0x7fffffffu && N % 256 == 0 && N <= 0x7fffffffu && K % 128 == 0
        && K / 128 <= PF_SCT_MAX && K * 2 * (size_t)M <= 0xffffffffull
        && ((uintptr_t)codes & 15) == 0 && ((uintptr_t)x & 15) == 0
        && ((uintptr_t)y & 15) == 0;
}

/* split-K partials: one device buffer, grown on demand, kept for the
 * process (launches on one device are stream-ordered users of it) */
static float *g_part;
static size_t g_part_cap;
#define GHIP_SPLITK_MAX_BYTES ((size_t)256 << 20)

extern "C" hipError_t ghip_launch_fp8_gemm(const uint8_t *codes, const float *scales,
                                           const uint16_t *x, uint16_t *y, size_t M,
                                           size_t N, size_t K, const uint32_t *exact_dev,
                                           uint32_t n_cu, const hipEvent_t *ev,
                                           hipStream_t st) {
    if (!ghip_fp8_gemm_fits(M, N, K, codes, x, y) || n_cu == 0 || n_cu % 8)
        return hipErrorInvalidValue;
    const size_t nblk = N / 256, nkb = K / 128;
    /* Tile height bm and K splits S: among bm in {256, 128, 64, 32} (no
     * taller than M needs) with the fewest splits that give 3/4 of the CUs
     * an item, the choice that moves the fewest bytes -- activation rows
     * (read once per column block), weights (once per row tile) and the
     * fp32 partials (written and read once per split). Splits keep >= 2 k
     * blocks each. When no choice reaches 3/4 of the CUs, the one with the
     * most items. */
    const size_t want = (size_t)n_cu * 3 / 4;
    uint32_t bm = 32, S = 1;
    size_t items = 0;
    {
        double best = -1.0;
        size_t best_items = 0;
        bool best_ok = false;
        for (uint32_t b = PF_BM; b >= 32; b >>= 1) {
            if (b > 32 && b / 2 >= M) continue;
            const size_t tiles = (M + b - 1) / b, base = tiles * nblk;
            size_t sp = 1;
            while (base * sp < want && sp + 1 <= nkb / 2
                   && (sp + 1) * M * N * sizeof(float) <= GHIP_SPLITK_MAX_BYTES)
                sp++;
            const size_t it = base * sp;
            const bool ok = it >= want;
            const double bytes = (double)nblk * tiles * b * K * 2 + (double)tiles * N * K
                               + (sp > 1 ? (double)sp * M * N * 8 : 0.0);
            const bool better = best < 0.0 || (ok && !best_ok)
                              || (ok == best_ok && (ok ? bytes < best : it > best_items));
            if (better) {
                best = bytes;
                best_items = it;
                best_ok = ok;
                bm = b;
                S = (uint32_t)sp;
            }
        }
        items = best_items;
    }
    if (S > 1) {
        const size_t need = (size_t)S * M * N * sizeof(float);
        if (need > g_part_cap) {
            if (g_part) (void)hipFree(g_part);
            g_part = nullptr;
            g_part_cap = 0;
            hipError_t e = hipMalloc((void **)&g_part, need);
            if (e != hipSuccess) return e;
            g_part_cap = need;
        }
    }
    /* XCD grid R x (8/R): fewest bytes into the 8 L2s, (8/R) |X| + R |W|,
     * among the grids that give every XCD the same number of units and of
     * column blocks (an uneven split would leave XCDs idle at the end) */
    uint32_t R = 0;
    {
        const size_t rows_u = ((M + bm - 1) / bm) * S;
        const double xb = (double)((M + bm - 1) / bm) * bm * K * 2, wb = (double)N * K;
        double best = -1.0;
        for (uint32_t r = 1; r <= 8; r <<= 1) {
            if (rows_u % r || nblk % (8 / r)) continue;
            const double b = (8.0 / r) * xb + r * wb;
            if (best < 0.0 || b < best) {
                best = b;
                R = r;
            }
        }
        if (!R) R = nblk >= 8 ? 1u : 8u;    /* no even grid: whole column blocks
                                                or whole units per XCD */
    }
    uint32_t g = items < n_cu ? (uint32_t)((items + 7) & ~(size_t)7) : n_cu;
    hipEvent_t e0 = ev ? ev[0] : nullptr, e1 = ev ? ev[1] : nullptr;
    GHIP_LAUNCH(e0, S > 1 ? nullptr : e1, k_fp8_gemm, dim3(g), dim3(256), PF_LDS, st, codes,
                scales, x, y, g_part, (uint32_t)M, (uint32_t)N, (uint32_t)K, bm, S, R,
                exact_dev);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const size_t n = M * N;                          /* N % 256 == 0: n % 4 == 0 */
    GHIP_LAUNCH(nullptr, e1, k_splitk_sum, dim3((uint32_t)((n / 4 + 255) / 256)), dim3(256),
                0, st, g_part, S, n, y);
    return hipGetLastError();
}

/* ------------------------------------------------------------------------ */
/* allocation-free prefill workspace                                        */
/* ------------------------------------------------------------------------ */

/* The workspace of apus_ghip_moe_prefill_dev_noalloc: a fixed device array
 * (each GPU the library runs on holds its own copy until the process
 * ends). Host code never passes `scratch` itself to a kernel (its name is a
 * host-side stand-in there): ghip_pf_scratch_init takes its device address
 * once per device, at the library's init, and every use goes through that
 * address. Every call on a GPU shares the array; calls that overlap in time
 * on one GPU race. */
static __device__ __align__(256) uint8_t scratch[GHIP_PF_SCRATCH_BYTES];
static void *g_scratch_dev[GHIP_MAX_DEVICES];

extern "C" hipError_t ghip_pf_scratch_init(int device) {
    if (device < 0 || device >= GHIP_MAX_DEVICES) return hipErrorInvalidDevice;
    if (g_scratch_dev[device]) return hipSuccess;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_dev[device] = p;
    return hipSuccess;
}

static size_t pf_up256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t ghip_pf_scratch_need(size_t pairs, uint32_t n_experts, uint32_t dim,
                                       uint32_t inter) {
    return pf_up256(PF_HDR_WORDS * sizeof(uint32_t))
         + pf_up256(ghip_moe_prefill_chunks(pairs) * n_experts * sizeof(uint32_t))
         + pf_up256(ghip_moe_prefill_max_tiles(pairs, n_experts) * 4 * sizeof(uint32_t))
         + 3 * pf_up256(pairs * sizeof(int32_t))
         + pf_up256(pairs * (size_t)inter * 2) + pf_up256(pairs * (size_t)dim * 2);
}

extern "C" hipError_t ghip_pf_scratch_ws(int device, size_t pairs, uint32_t n_experts,
                                         uint32_t dim, uint32_t inter, uint32_t n_cu,
                                         GhipMoePrefillWs *ws) {
    if (device < 0 || device >= GHIP_MAX_DEVICES || !g_scratch_dev[device])
        return hipErrorNotInitialized;
    if (ghip_pf_scratch_need(pairs, n_experts, dim, inter) > GHIP_PF_SCRATCH_BYTES)
        return hipErrorOutOfMemory;
    uint8_t *b = (uint8_t *)g_scratch_dev[device];
    size_t o = 0;
    auto take = [&](size_t n) {
        uint8_t *p = b + o;
        o += pf_up256(n);
        return (void *)p;
    };
    ws->hdr = (uint32_t *)take(PF_HDR_WORDS * sizeof(uint32_t));
    ws->cnt = (uint32_t *)take(ghip_moe_prefill_chunks(pairs) * n_experts * sizeof(uint32_t));
    ws->tiles = (uint32_t *)take(ghip_moe_prefill_max_tiles(pairs, n_experts) * 16);
    ws->eid = (int32_t *)take(pairs * sizeof(int32_t));
    ws->perm = (int32_t *)take(pairs * sizeof(int32_t));
    ws->pos = (int32_t *)take(pairs * sizeof(int32_t));
    ws->h = (uint16_t *)take(pairs * (size_t)inter * 2);
    ws->o = (uint16_t *)take(pairs * (size_t)dim * 2);
    ws->cap_pairs = pairs;
    ws->n_cu = n_cu;
    return hipSuccess;
}

extern "C" hipError_t ghip_moe_prefill_init(void) {
    const void *ks[5] = {(const void *)k_pf_gemm<0, 8>, (const void *)k_pf_gemm<0, 4>,
                         (const void *)k_pf_gemm<1, 8>, (const void *)k_pf_gemm<1, 4>,
                         (const void *)k_fp8_gemm};
    const int lds[5] = {PF_LDS_WB, PF_LDS, PF_LDS_WB, PF_LDS, PF_LDS};
    for (int i = 0; i < 5; i++) {
        hipError_t e = hipFuncSetAttribute(ks[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                           lds[i]);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
