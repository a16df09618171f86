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
 *   k_pf_gemm<0>  gate/up: H[s] = SwiGLU(bf16(x Wg^T), bf16(x Wu^T)) for the
 *                 sorted pair rows s of each tile; x rows gathered by token.
 *   k_pf_gemm<1>  down: O[s] = bf16(H[s] Wd^T).
 *   k_pf_combine  out[t] = ascending-expert, bf16-per-add sum of
 *                 bf16(O[s] * w) over the token's pairs (c/gmoe.h:307-320).
 *
 * GEMM tile (both modes). A workgroup of 4 waves owns one tile of up to 256
 * expert-sorted rows and one column block; K is walked in 128-wide steps,
 * one F32 scale block. Each wave owns two 32-column weight slots (gate and
 * up columns [c, c+32) in mode 0, so the SwiGLU epilogue is lane-local; two
 * 128-apart down column groups in mode 1) for all tile rows, accumulating
 * 2 x 8 v_mfma_f32_32x32x16_bf16 blocks (256 fp32 per lane) in AGPRs.
 * FP8 weights go straight from HBM into registers in the MFMA B layout
 * (lane (n, h) holds weight row n, codes [64h, 64h+64) of the step) and are
 * dequantized there, bit-exact (bf16_rne(e4m3 * scale), c/fp8blk.h:115-136).
 * The activation tile is gathered into LDS, double-buffered, one barrier
 * per step. MFMA k-step s takes codes [64h + 8s, +8) of lane half h and the
 * A operand is read with the same mapping: a permutation of k inside the
 * 128-block, identical for A and B. 32-row blocks past the tile's row count
 * skip their MFMAs, so ragged experts cost what their rows need.
 *
 * Workgroup -> work mapping is XCD-aware: hardware deals workgroups to the
 * 8 XCDs round-robin, so block b is remapped to logical id
 * (b % 8) * (G / 8) + b / 8 and logical ids enumerate column blocks fastest:
 * the column blocks of one tile (same gathered activation rows) run on one
 * XCD and share its L2.
 */
#include "ghip_device.h"
#include "ghip_internal.h"

typedef float ghip_f32x16 __attribute__((ext_vector_type(16)));

#define PF_CHUNK 1024            /* pairs per permutation workgroup */
#define PF_BM 256                /* rows per GEMM tile */
#define PF_RB (PF_BM / 32)       /* 32-row MFMA blocks per tile */
#define PF_PITCH 136             /* LDS row pitch (bf16): 128 + 8 pad */
#define PF_BUF (PF_BM * PF_PITCH)
#define PF_MAXK 16               /* max top-k per token */
#define PF_MAXE 1024             /* max experts in a bank */

/* ------------------------------------------------------------------------ */
/* permutation                                                              */
/* ------------------------------------------------------------------------ */

/* One workgroup per PF_CHUNK pairs (pair p = t * topk + j). eid[p] = the
 * expert of p, or -1 when the id is out of range (flags hdr[PF_HDR_ERR]) or
 * repeats an earlier slot of the same token. cnt[chunk][e] = count. */
__global__ __launch_bounds__(1024) void k_pf_count(
    const int32_t *__restrict__ idx, uint32_t P, uint32_t topk, uint32_t E,
    uint32_t *__restrict__ cnt, int32_t *__restrict__ eid,
    uint32_t *__restrict__ hdr) {
    extern __shared__ uint32_t hist[];
    for (uint32_t i = threadIdx.x; i < E; i += 1024) hist[i] = 0;
    __syncthreads();
    const uint32_t p = blockIdx.x * PF_CHUNK + threadIdx.x;
    if (p < P) {
        const int32_t e = idx[p];
        const uint32_t t = p / topk, j = p - t * topk;
        bool ok = e >= 0 && (uint32_t)e < E;
        if (!ok) {
            atomicOr(&hdr[PF_HDR_ERR], 1u);
        } else {
            for (uint32_t jj = 0; jj < j; jj++)
                if (idx[(size_t)t * topk + jj] == e) { ok = false; break; }
        }
        eid[p] = ok ? e : -1;
        if (ok) atomicAdd(&hist[e], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < E; i += 1024)
        cnt[(size_t)blockIdx.x * E + i] = hist[i];
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
 * expert); tiles[] = {expert, first sorted row, rows, 0}; hdr gets the tile
 * count and the number of valid pairs. */
__global__ __launch_bounds__(1024) void k_pf_scan(
    uint32_t *__restrict__ cnt, uint32_t nch, uint32_t E,
    uint4 *__restrict__ tiles, uint32_t *__restrict__ hdr) {
    __shared__ uint32_t sh[16];
    const uint32_t e = threadIdx.x;
    uint32_t tot = 0;
    if (e < E)
        for (uint32_t c = 0; c < nch; c++) {
            const uint32_t v = cnt[(size_t)c * E + e];
            cnt[(size_t)c * E + e] = tot;
            tot += v;
        }
    const uint32_t nt = (tot + PF_BM - 1) / PF_BM;
    const uint32_t base = pf_block_scan(tot, sh) - tot;
    const uint32_t tb = pf_block_scan(nt, sh) - nt;
    if (e < E) {
        for (uint32_t c = 0; c < nch; c++) cnt[(size_t)c * E + e] += base;
        for (uint32_t i = 0; i < nt; i++) {
            const uint32_t r0 = i * PF_BM;
            const uint32_t rows = tot - r0 < PF_BM ? tot - r0 : PF_BM;
            tiles[tb + i] = make_uint4(e, base + r0, rows, 0u);
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

/* 8 codes (two dwords) -> one bf16x8 MFMA operand. `exact` (wave-uniform:
 * the expert holds NaN codes) selects the integer decode; a branch per
 * operand keeps one copy of the MFMA loop and its registers. */
__device__ __forceinline__ ghip_bf16x8 pf_deq8(uint32_t d0, uint32_t d1, float s,
                                               bool exact) {
    ghip_u32x2 a, b;
    if (exact) {
        a = ghip_deq4<true>(d0, s);
        b = ghip_deq4<true>(d1, s);
    } else {
        a = ghip_deq4<false>(d0, s);
        b = ghip_deq4<false>(d1, s);
    }
    ghip_u32x4 v = {a[0], a[1], b[0], b[1]};
    return __builtin_bit_cast(ghip_bf16x8, v);
}

/* One 128-wide k step of a wave: 8 MFMA k-slices x (up to) 8 row blocks x
 * 2 weight slots. */
__device__ __forceinline__ void pf_step(const uint16_t *__restrict__ ab,
                                        const ghip_u32x4 (&c0)[4],
                                        const ghip_u32x4 (&c1)[4], float s0,
                                        float s1, uint32_t nrb, uint32_t n,
                                        uint32_t h, bool exact,
                                        ghip_f32x16 (&a0)[PF_RB],
                                        ghip_f32x16 (&a1)[PF_RB]) {
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const ghip_u32x4 q0 = c0[s >> 1], q1 = c1[s >> 1];
        const int o = (s & 1) * 2;
        const ghip_bf16x8 b0 = pf_deq8(q0[o], q0[o + 1], s0, exact);
        const ghip_bf16x8 b1 = pf_deq8(q1[o], q1[o + 1], s1, exact);
        const uint16_t *ar = ab + n * PF_PITCH + 64 * h + 8 * s;
#pragma unroll
        for (int rb = 0; rb < PF_RB; rb++) {
            if ((uint32_t)rb < nrb) {
                const ghip_bf16x8 a =
                    *(const ghip_bf16x8 *)(ar + (size_t)rb * 32 * PF_PITCH);
                a0[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b0, a0[rb], 0, 0, 0);
                a1[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b1, a1[rb], 0, 0, 0);
            }
        }
    }
}

/* MODE 0: act = x [T, dim], rows gathered by token (perm[s] / topk);
 *         out = H [P, inter] (sorted rows), SwiGLU epilogue.
 * MODE 1: act = H [P, inter] (sorted rows); out = O [P, dim] (sorted rows),
 *         bf16 expert outputs.
 * Grid: G (multiple of 8) >= tiles * nblk; 256 threads. */
template <int MODE>
__global__ __launch_bounds__(256, 1) void k_pf_gemm(
    GhipBank bank, const uint16_t *__restrict__ act,
    const int32_t *__restrict__ perm, const uint4 *__restrict__ tiles,
    const uint32_t *__restrict__ hdr, uint32_t nblk, uint32_t topk,
    float limit, uint16_t *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t L = (b & 7u) * (G >> 3) + (b >> 3);
    const uint32_t tile = L / nblk, nb = L - tile * nblk;
    if (tile >= hdr[PF_HDR_NTILES]) return;
    const uint4 td = tiles[tile];
    const uint32_t e = td.x, row0 = td.y, rows = td.z;
    const uint32_t K = MODE == 0 ? bank.dim : bank.inter;
    const uint32_t nkb = K >> 7;
    const uint8_t *slab = bank.base + (size_t)e * bank.stride;
    const uint32_t tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const uint32_t n = lane & 31, h = lane >> 5;
    uint32_t col0, col1;
    const uint8_t *w0, *w1;
    const float *s0, *s1;
    if (MODE == 0) {
        col0 = col1 = nb * 128 + 32 * wv;
        w0 = slab + bank.off_gw;
        w1 = slab + bank.off_uw;
        s0 = (const float *)(slab + bank.off_gs);
        s1 = (const float *)(slab + bank.off_us);
    } else {
        col0 = nb * 256 + 32 * wv;
        col1 = col0 + 128;
        w0 = w1 = slab + bank.off_dw;
        s0 = s1 = (const float *)(slab + bank.off_ds);
    }
    const uint8_t *wr0 = w0 + (size_t)(col0 + n) * K + 64 * h;
    const uint8_t *wr1 = w1 + (size_t)(col1 + n) * K + 64 * h;
    const float *sr0 = s0 + (size_t)(col0 >> 7) * nkb;
    const float *sr1 = s1 + (size_t)(col1 >> 7) * nkb;
    const bool exact = bank.nan_flags && bank.nan_flags[e];
    const uint32_t nrb = (rows + 31) >> 5;

    /* activation rows of this thread's 16 loads: tile row i*16 + tid/16,
     * 16-byte piece tid%16 of the 128-wide step; rows past the tile clamp
     * to its last row (computed, never stored). */
    uint32_t arow[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        uint32_t r = i * 16 + (tid >> 4);
        r = r < rows ? r : rows - 1;
        arow[i] = MODE == 0 ? (uint32_t)perm[row0 + r] / topk : row0 + r;
    }
    const uint32_t pc = (tid & 15) * 8;
    const uint32_t nld = nrb * 2;         /* 16-row groups that hold rows */

    ghip_u32x4 areg[16];
    ghip_u32x4 c0[4], c1[4], n0[4], n1[4];
#pragma unroll
    for (int i = 0; i < 16; i++)
        if ((uint32_t)i < nld)
            areg[i] = *(const ghip_u32x4 *)(act + (size_t)arow[i] * K + pc);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        c0[q] = __builtin_nontemporal_load((const ghip_u32x4 *)(wr0 + 16 * q));
        c1[q] = __builtin_nontemporal_load((const ghip_u32x4 *)(wr1 + 16 * q));
    }
#pragma unroll
    for (int i = 0; i < 16; i++)
        if ((uint32_t)i < nld)
            *(ghip_u32x4 *)(lds + (i * 16 + (tid >> 4)) * PF_PITCH + pc) = areg[i];
    __syncthreads();

    ghip_f32x16 a0[PF_RB], a1[PF_RB];
#pragma unroll
    for (int rb = 0; rb < PF_RB; rb++)
#pragma unroll
        for (int i = 0; i < 16; i++) { a0[rb][i] = 0.0f; a1[rb][i] = 0.0f; }

    for (uint32_t kb = 0; kb < nkb; kb++) {
        const uint32_t kn = kb + 1 < nkb ? kb + 1 : kb;   /* clamped prefetch */
#pragma unroll
        for (int i = 0; i < 16; i++)
            if ((uint32_t)i < nld)
                areg[i] = *(const ghip_u32x4 *)(act + (size_t)arow[i] * K +
                                                 (size_t)kn * 128 + pc);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            n0[q] = __builtin_nontemporal_load(
                (const ghip_u32x4 *)(wr0 + (size_t)kn * 128 + 16 * q));
            n1[q] = __builtin_nontemporal_load(
                (const ghip_u32x4 *)(wr1 + (size_t)kn * 128 + 16 * q));
        }
        const float sc0 = sr0[kb], sc1 = sr1[kb];
        const uint16_t *ab = lds + (kb & 1) * PF_BUF;
        pf_step(ab, c0, c1, sc0, sc1, nrb, n, h, exact, a0, a1);
        if (kb + 1 < nkb) {
            uint16_t *nbuf = lds + ((kb + 1) & 1) * PF_BUF;
#pragma unroll
            for (int i = 0; i < 16; i++)
                if ((uint32_t)i < nld)
                    *(ghip_u32x4 *)(nbuf + (i * 16 + (tid >> 4)) * PF_PITCH + pc) = areg[i];
        }
#pragma unroll
        for (int q = 0; q < 4; q++) { c0[q] = n0[q]; c1[q] = n1[q]; }
        __syncthreads();
    }

    /* epilogue: lane (n, h), register i of row block rb holds output row
     * rb*32 + 8*(i/4) + 4*h + i%4, column n of each slot */
    const uint32_t N = MODE == 0 ? bank.inter : bank.dim;
#pragma unroll
    for (int rb = 0; rb < PF_RB; rb++) {
        if ((uint32_t)rb >= nrb) break;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t r = rb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
            if (r < rows) {
                uint16_t *o = out + (size_t)(row0 + r) * N;
                if (MODE == 0) {
                    const float g = ghip_bf16_round(a0[rb][i]);
                    const float u = ghip_bf16_round(a1[rb][i]);
                    o[col0 + n] = (uint16_t)ghip_swiglu(g, u, limit);
                } else {
                    o[col0 + n] = (uint16_t)ghip_bf16_bits(a0[rb][i]);
                    o[col1 + n] = (uint16_t)ghip_bf16_bits(a1[rb][i]);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ordered combine                                                          */
/* ------------------------------------------------------------------------ */

/* One thread per 8 output columns of one token: the token's kept pairs in
 * ascending expert id, contrib = bf16(bf16(o) * w), y = bf16(y + contrib),
 * y from +0 (c/gmoe.h:307-320). */
__global__ __launch_bounds__(256) void k_pf_combine(
    const uint16_t *__restrict__ O, const int32_t *__restrict__ pos,
    const int32_t *__restrict__ idx, const float *__restrict__ w, uint32_t T,
    uint32_t topk, uint32_t dim, uint16_t *__restrict__ out) {
    const uint32_t per = dim >> 3;
    const size_t gid = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t t = gid / per;
    if (t >= T) return;
    const uint32_t d = (uint32_t)(gid - t * per) * 8;
    int32_t ke[PF_MAXK], ks[PF_MAXK];
    float kw[PF_MAXK];
#pragma unroll
    for (int j = 0; j < PF_MAXK; j++) {
        const bool v = (uint32_t)j < topk;
        const size_t p = t * topk + j;
        const int32_t s = v ? pos[p] : -1;
        ke[j] = s >= 0 ? idx[p] : 0x7fffffff;
        ks[j] = s;
        kw[j] = v ? w[p] : 0.0f;
    }
    float y[8];
#pragma unroll
    for (int q = 0; q < 8; q++) y[q] = 0.0f;
    int32_t prev = -1;
    for (uint32_t r = 0; r < topk; r++) {
        int32_t best = 0x7fffffff, bs = -1;
        float bw = 0.0f;
#pragma unroll
        for (int j = 0; j < PF_MAXK; j++)
            if (ke[j] > prev && ke[j] < best) { best = ke[j]; bs = ks[j]; bw = kw[j]; }
        if (bs < 0) break;
        prev = best;
        const ghip_u32x4 v = *(const ghip_u32x4 *)(O + (size_t)bs * dim + d);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const uint32_t bits = (v[q >> 1] >> (16 * (q & 1))) & 0xffffu;
            const float c = ghip_bf16_round(ghip_bf16_f32(bits) * bw);
            y[q] = ghip_bf16_round(y[q] + c);
        }
    }
    ghip_u32x4 r;
#pragma unroll
    for (int q = 0; q < 4; q++)
        r[q] = ghip_bf16_bits(y[2 * q]) | (ghip_bf16_bits(y[2 * q + 1]) << 16);
    *(ghip_u32x4 *)(out + t * dim + d) = r;
}

/* ------------------------------------------------------------------------ */

extern "C" size_t ghip_moe_prefill_max_tiles(size_t pairs, uint32_t n_experts) {
    return (pairs + PF_BM - 1) / PF_BM + n_experts;
}

extern "C" size_t ghip_moe_prefill_chunks(size_t pairs) {
    return (pairs + PF_CHUNK - 1) / PF_CHUNK;
}

static size_t round8(size_t v) { return (v + 7) & ~(size_t)7; }

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
    if (topk <= 0 || topk > PF_MAXK || E == 0 || E > PF_MAXE)
        return hipErrorInvalidValue;
    if (dim == 0 || inter == 0 || dim % 256 || inter % 128) return hipErrorInvalidValue;
    const size_t P = T * (size_t)topk;
    if (P > ws->cap_pairs || P > 0x7fffffffu) return hipErrorInvalidValue;
    if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)bank->base & 15)
        || (bank->stride & 15) || (bank->off_gw & 15) || (bank->off_uw & 15)
        || (bank->off_dw & 15) || (bank->off_gs & 3) || (bank->off_us & 3)
        || (bank->off_ds & 3))
        return hipErrorInvalidValue;
    const uint32_t nch = (uint32_t)ghip_moe_prefill_chunks(P);
    const size_t mt = ghip_moe_prefill_max_tiles(P, E);
    hipEvent_t e0 = ev ? ev[0] : nullptr, e1 = ev ? ev[1] : nullptr;
    hipEvent_t e2 = ev ? ev[2] : nullptr, e3 = ev ? ev[3] : nullptr;
    hipEvent_t e4 = ev ? ev[4] : nullptr, e5 = ev ? ev[5] : nullptr;
    hipEvent_t e6 = ev ? ev[6] : nullptr, e7 = ev ? ev[7] : nullptr;
    hipError_t e;
    if ((e = ghip_launch_fill_u32(ws->hdr, PF_HDR_WORDS, 0u, st)) != hipSuccess) return e;
    GHIP_LAUNCH(e0, nullptr, k_pf_count, dim3(nch), dim3(1024), E * 4, st, idx,
                (uint32_t)P, (uint32_t)topk, E, ws->cnt, ws->eid, ws->hdr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_pf_scan, dim3(1), dim3(1024), 0, st, ws->cnt, nch, E,
                       (uint4 *)ws->tiles, ws->hdr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GHIP_LAUNCH(nullptr, e1, k_pf_scatter, dim3(nch), dim3(1024), 16 * E * 4, st,
                ws->eid, (uint32_t)P, E, ws->cnt, ws->perm, ws->pos);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t lds = 2 * (size_t)PF_BUF * 2;
    const size_t g0 = round8(mt * (inter / 128)), g1 = round8(mt * (dim / 256));
    if (g0 > 0x7fffffffu || g1 > 0x7fffffffu) return hipErrorInvalidValue;
    GHIP_LAUNCH(e2, e3, k_pf_gemm<0>, dim3((uint32_t)g0), dim3(256), lds, st, *bank,
                x, ws->perm, (const uint4 *)ws->tiles, ws->hdr, inter / 128,
                (uint32_t)topk, limit, ws->h);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    GHIP_LAUNCH(e4, e5, k_pf_gemm<1>, dim3((uint32_t)g1), dim3(256), lds, st, *bank,
                ws->h, ws->perm, (const uint4 *)ws->tiles, ws->hdr, dim / 256,
                (uint32_t)topk, limit, ws->o);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t nthr = T * (size_t)(dim / 8);
    GHIP_LAUNCH(e6, e7, k_pf_combine, dim3((uint32_t)((nthr + 255) / 256)), dim3(256),
                0, st, ws->o, ws->pos, idx, w, (uint32_t)T, (uint32_t)topk, dim, out);
    return hipGetLastError();
}

extern "C" hipError_t ghip_moe_prefill_init(void) {
    const int lds = 2 * PF_BUF * 2;
    hipError_t e = hipFuncSetAttribute((const void *)k_pf_gemm<0>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void *)k_pf_gemm<1>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, lds);
}
