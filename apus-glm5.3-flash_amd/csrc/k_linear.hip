/*
 * k_linear.hip — gfx950 kernels for the dense FP8-block path:
 *   K1  k_dequant16 / k_dequant_any : FP8-E4M3 + F32 128x128 scales -> BF16,
 *       bit-exact vs c/fp8blk.h:115-136 (apus_fp8blk_rows_scalar).
 *   K2  k_fp8_gemv : decode / MTP-verify GEMV (M <= 4 per launch) with the
 *       dequant fused in registers and the k reduction on MFMA
 *       (v_mfma_f32_16x16x32_bf16), the composition of c/gdsa.h:525-534
 *       (dequant -> bf16 -> fp32-accumulated GEMM -> RNE bf16).
 *   k_fp8_linear_any / k_bf16_linear_any : shape-general fallbacks (ceil
 *       shapes, K not a multiple of 64) with the exact integer decode.
 *   k_nan_scan : flags the out-of-contract NaN codes 0x7F/0xFF so callers
 *       can select the exact decode for such weights.
 *
 * GEMV tiling (K2). A workgroup owns 16 consecutive output rows; its NW
 * waves split K into 128-wide chunks (one scale block; wave w takes chunks
 * w, w+NW, ...). Per chunk, lane l loads 32 codes of row (l % 16) at k
 * offset 32*(l / 16) (two 16-byte loads; a wave covers 16 full 128-byte
 * lines), dequantizes them to four bf16x8 operands and issues four MFMAs
 * whose A operand is x staged in LDS. The MFMA k-slot
 * to k mapping is any permutation used identically for A and B, so the
 * result is an exact-product fp32 sum in a different order than the
 * reference's sequential k: a tolerance-class result, per the contract.
 * Partial sums of the NW waves are combined in LDS in a fixed order, so the
 * output is deterministic run to run.
 */
#include "ghip_device.h"
#include <type_traits>
#include "ghip_internal.h"

#define GEMV_NW 8          /* waves per workgroup (k split) */
#define GEMV_U 4           /* 128-wide chunks (2 loads each) per batch */

/* ------------------------------------------------------------------------ */
/* K1: dequant                                                              */
/* ------------------------------------------------------------------------ */

/* K % 16 == 0: one thread per 16 consecutive codes of a row (they share
 * one 128-block scale because 16 divides 128). */
template <bool EXACT>
__global__ __launch_bounds__(256) void k_dequant16(
    const uint8_t *__restrict__ w, const float *__restrict__ s,
    uint16_t *__restrict__ out, uint32_t O, uint32_t K, uint32_t nkb) {
    const uint32_t cpr = K >> 4;                       /* chunks per row */
    const size_t n = (size_t)O * cpr;
    for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < n;
         c += (size_t)gridDim.x * 256) {
        uint32_t o = (uint32_t)(c / cpr);
        uint32_t k0 = (uint32_t)(c - (size_t)o * cpr) << 4;
        float sc = s[(size_t)(o >> 7) * nkb + (k0 >> 7)];
        ghip_u32x4 v = *(const ghip_u32x4 *)(w + (size_t)o * K + k0);
        ghip_u32x4 r0, r1;
        ghip_deq16_u32<EXACT>(v, sc, r0, r1);
        ghip_u32x4 *dst = (ghip_u32x4 *)(out + (size_t)o * K + k0);
        dst[0] = r0;
        dst[1] = r1;
    }
}

/* Any K: one thread per element, exact integer path. */
__global__ __launch_bounds__(256) void k_dequant_any(
    const uint8_t *__restrict__ w, const float *__restrict__ s,
    uint16_t *__restrict__ out, uint32_t O, uint32_t K, uint32_t nkb) {
    const size_t n = (size_t)O * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (size_t)gridDim.x * 256) {
        uint32_t o = (uint32_t)(i / K), k = (uint32_t)(i - (size_t)o * K);
        float sc = s[(size_t)(o >> 7) * nkb + (k >> 7)];
        out[i] = (uint16_t)ghip_bf16_bits(ghip_e4m3_exact(w[i]) * sc);
    }
}

/* NaN-code scan: bytes whose low 7 bits are all ones (0x7F / 0xFF). */
__global__ __launch_bounds__(256) void k_nan_scan(
    const uint8_t *__restrict__ p, size_t n, uint32_t *flag) {
    const size_t nv = n >> 4;
    uint32_t hit = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < nv;
         i += (size_t)gridDim.x * 256) {
        ghip_u32x4 v = *(const ghip_u32x4 *)(p + (i << 4));
        for (int j = 0; j < 4; j++)
            hit |= ((v[j] & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
    }
    if (blockIdx.x == 0)
        for (size_t i = (nv << 4) + threadIdx.x; i < n; i += 256)
            hit |= ((p[i] & 0x7fu) == 0x7fu);
    if (hit) atomicOr(flag, 1u);
}

/* ------------------------------------------------------------------------ */
/* K2: FP8 GEMV, M <= 4, K % 128 == 0                                       */
/* ------------------------------------------------------------------------ */

/* One batch of a wave's chunk loads: chunks c0, c0 + NW, ... (GEMV_U of
 * them). The first batch is issued before x is staged so the two latencies
 * overlap. */
__device__ __forceinline__ void gemv16_fetch(const uint8_t *__restrict__ wr,
                                             uint32_t nch, uint32_t c0,
                                             ghip_chunk *buf) {
    /* unconditional (chunk clamped; the compute loop skips c >= nch) so the
     * waitcnt pass sees a fixed number of loads */
#pragma unroll
    for (int u = 0; u < GEMV_U; u++) {
        uint32_t c = min(c0 + u * GEMV_NW, nch - 1u);
        buf[u] = ghip_chunk_load(wr + (size_t)c * 128);
    }
}

/* buf holds the first batch on entry and is refilled in place. */
/* sc holds the first batch's scales (fetched with the weights). */
template <bool EXACT>
__device__ __forceinline__ ghip_f32x4 gemv16_rows(
    const uint8_t *__restrict__ wr, const float *__restrict__ srow,
    const uint16_t *xa, uint32_t nch, uint32_t wv, ghip_chunk (&buf)[GEMV_U],
    const float (&sc)[GEMV_U]) {
    ghip_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c0 = wv; c0 < nch; c0 += GEMV_NW * GEMV_U) {
        float s2[GEMV_U];
        if (c0 != wv) {
            gemv16_fetch(wr, nch, c0, buf);
#pragma unroll
            for (int u = 0; u < GEMV_U; u++) s2[u] = srow[min(c0 + u * GEMV_NW, nch - 1u)];
        } else {
#pragma unroll
            for (int u = 0; u < GEMV_U; u++) s2[u] = sc[u];
        }
#pragma unroll
        for (int u = 0; u < GEMV_U; u++) {
            uint32_t c = c0 + u * GEMV_NW;
            if (c < nch) ghip_chunk_mfma<EXACT>(buf[u], s2[u], xa + c * 128, acc);
        }
    }
    return acc;
}

template <int M>
__global__ __launch_bounds__(GEMV_NW * 64, 4) void k_fp8_gemv(
    const uint8_t *__restrict__ W, const float *__restrict__ S,
    const uint16_t *__restrict__ X, uint16_t *__restrict__ Y, uint32_t O,
    uint32_t K, uint32_t nkb, const uint32_t *__restrict__ exact_flag) {
    extern __shared__ __align__(16) uint16_t xs[];     /* M x K */
    __shared__ float red[GEMV_NW][M][16];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t row0 = blockIdx.x * 16u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t row = min(row0 + n, O - 1u);
    const uint8_t *wr = W + (size_t)row * K + 32u * g;
    const uint32_t nch = K >> 7;
    /* this wave's x slices first, then the weights, then the slices into
     * LDS (ghip_wstage_*: no workgroup barrier) */
    ghip_stage stx;
    ghip_wstage_load(stx, X, M, K, nch, wv, GEMV_NW, lane);
    ghip_chunk pre[GEMV_U];
    gemv16_fetch(wr, nch, wv, pre);
    const float *srow = S + (size_t)(row0 >> 7) * nkb;
    float sc[GEMV_U];
#pragma unroll
    for (int u = 0; u < GEMV_U; u++) sc[u] = srow[min(wv + u * GEMV_NW, nch - 1u)];
    const bool exact = exact_flag != nullptr && *exact_flag != 0u;
    ghip_wstage_store(stx, xs, X, M, K, nch, wv, GEMV_NW, lane);
    /* MFMA A row i = lane % 16 is token m; rows m >= M only feed output
     * rows that are discarded, so they read row M-1 instead of zeros. */
    const uint16_t *xa = xs + (size_t)min(n, (uint32_t)M - 1u) * K + 32u * g;
    ghip_f32x4 acc = exact ? gemv16_rows<true>(wr, srow, xa, nch, wv, pre, sc)
                           : gemv16_rows<false>(wr, srow, xa, nch, wv, pre, sc);
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < M; i++) red[wv][i][n] = acc[i];
    }
    __syncthreads();
    if (tid < (uint32_t)M * 16u) {
        uint32_t m = tid >> 4, nn = tid & 15u;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < GEMV_NW; w++) s += red[w][m][nn];
        if (row0 + nn < O) Y[(size_t)m * O + row0 + nn] = (uint16_t)ghip_bf16_bits(s);
    }
}

/* ------------------------------------------------------------------------ */
/* shape-general fallbacks: one wave per (row, m), exact decode             */
/* ------------------------------------------------------------------------ */

__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__global__ __launch_bounds__(256) void k_fp8_linear_any(
    const uint8_t *__restrict__ W, const float *__restrict__ S,
    const uint16_t *__restrict__ X, uint16_t *__restrict__ Y, uint32_t M,
    uint32_t O, uint32_t K, uint32_t nkb) {
    const uint32_t lane = threadIdx.x & 63u;
    const size_t item = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (size_t)M * O) return;
    const uint32_t m = (uint32_t)(item / O), o = (uint32_t)(item - (size_t)m * O);
    const uint8_t *wr = W + (size_t)o * K;
    const float *srow = S + (size_t)(o >> 7) * nkb;
    const uint16_t *xr = X + (size_t)m * K;
    float acc = 0.0f;
    for (uint32_t k = lane; k < K; k += 64) {
        float wv = ghip_bf16_round(ghip_e4m3_exact(wr[k]) * srow[k >> 7]);
        acc += wv * ghip_bf16_f32(xr[k]);
    }
    acc = wave_sum(acc);
    if (lane == 0) Y[(size_t)m * O + o] = (uint16_t)ghip_bf16_bits(acc);
}

__global__ __launch_bounds__(256) void k_bf16_linear_any(
    const uint16_t *__restrict__ W, const uint16_t *__restrict__ X,
    uint16_t *__restrict__ Y, uint32_t M, uint32_t O, uint32_t K) {
    const uint32_t lane = threadIdx.x & 63u;
    const size_t item = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (size_t)M * O) return;
    const uint32_t m = (uint32_t)(item / O), o = (uint32_t)(item - (size_t)m * O);
    const uint16_t *wr = W + (size_t)o * K;
    const uint16_t *xr = X + (size_t)m * K;
    float acc = 0.0f;
    for (uint32_t k = lane; k < K; k += 64)
        acc += ghip_bf16_f32(wr[k]) * ghip_bf16_f32(xr[k]);
    acc = wave_sum(acc);
    if (lane == 0) Y[(size_t)m * O + o] = (uint16_t)ghip_bf16_bits(acc);
}

/* ------------------------------------------------------------------------ */
/* launchers                                                                */
/* ------------------------------------------------------------------------ */

static uint32_t grid_for(size_t items, size_t per_block, uint32_t cap) {
    size_t g = (items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (uint32_t)g;
}

extern "C" hipError_t ghip_launch_dequant(const uint8_t *codes,
                                          const float *scales, uint16_t *out,
                                          size_t O, size_t K, int exact,
                                          hipStream_t st) {
    if (O == 0 || K == 0) return hipSuccess;
    if (O > 0xffffffffu || K > 0xffffffffu) return hipErrorInvalidValue;
    uint32_t nkb = (uint32_t)((K + 127) / 128);
    bool aligned = (K % 16 == 0) && (((uintptr_t)codes & 15) == 0)
                && (((uintptr_t)out & 15) == 0);
    if (aligned) {
        uint32_t g = grid_for(O * (K / 16), 256, 65536);
        if (exact)
            hipLaunchKernelGGL(k_dequant16<true>, dim3(g), dim3(256), 0, st,
                               codes, scales, out, (uint32_t)O, (uint32_t)K, nkb);
        else
            hipLaunchKernelGGL(k_dequant16<false>, dim3(g), dim3(256), 0, st,
                               codes, scales, out, (uint32_t)O, (uint32_t)K, nkb);
    } else {
        uint32_t g = grid_for(O * K, 256, 65536);
        hipLaunchKernelGGL(k_dequant_any, dim3(g), dim3(256), 0, st, codes,
                           scales, out, (uint32_t)O, (uint32_t)K, nkb);
    }
    return hipGetLastError();
}

extern "C" hipError_t ghip_launch_nan_scan(const uint8_t *codes, size_t n,
                                           uint32_t *flag, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (((uintptr_t)codes & 15) != 0) return hipErrorInvalidValue;
    uint32_t g = grid_for(n / 16 + 1, 256 * 8, 4096);
    hipLaunchKernelGGL(k_nan_scan, dim3(g), dim3(256), 0, st, codes, n, flag);
    return hipGetLastError();
}

/* ------------------------------------------------------------------------ */
/* K2 streaming: persistent FP8 / BF16 GEMV, register-load chunk streams   */
/* ------------------------------------------------------------------------ */

#define GS_NW 8                  /* waves per workgroup */
/* LDS chunk slots per wave: a chunk is written from registers and read
 * back in the MFMA layout while the next ones are in flight: two for FP8
 * weights (measured: one 13.8 us, two 12.3, three 12.6 on config 1), three
 * for BF16 (the LM head: two 226 us, three 208) */
#define GS_R 3
#define GS_LDS (144u * 1024u)    /* dynamic LDS limit of the streaming GEMV */

/* Y[m, rows] for M <= 4 token rows. A row group (16 weight rows) is split
 * over KS waves along K (KS in {2, 8}); a workgroup pass covers 8 / KS row
 * groups, passes run over the groups persistently (grid <= CUs). Each wave
 * streams its chunks (16 rows x 128 bytes: 128 FP8 codes with one scale
 * block, or 64 BF16 weights when BF) through registers: two 16-byte loads
 * per lane in a whole-line pattern (load i: rows 8i + lane / 8, piece lane
 * % 8), two chunks in flight, each chunk written to a wave-private 2-slot
 * LDS area (lane l's bytes at 16 l, piece p of row r at p ^ ((r >> 1) & 7))
 * and read back in the MFMA layout, dequantized in registers (FP8) and
 * reduced on MFMA with the token rows of x (staged once per workgroup) as
 * the A operand: A row i = lane % 16 is token min(i, M-1), rows past M feed
 * output rows that are discarded. The KS partial sums of a group are added
 * in LDS in a fixed order (deterministic). BF: the BF16 GEMV of the
 * bf16_gemm hook (c/bf16.h:712-767), no scales; lane 16g + n holds row n,
 * weights [16g, 16g + 16) of the chunk, two v_mfma_f32_16x16x32_bf16 with
 * x at the same k. */
template <int M, int KS, bool BF = false>
__global__ __launch_bounds__(GS_NW * 64, 1) void k_fp8_gemv_stream(
    const uint8_t *__restrict__ W, const float *__restrict__ S,
    const uint16_t *__restrict__ X, uint16_t *__restrict__ Y, uint32_t O,
    uint32_t K, const uint32_t *__restrict__ exact_flag) {
    constexpr uint32_t GPP = GS_NW / KS;             /* row groups per pass */
    extern __shared__ __attribute__((aligned(1024))) uint8_t gsl[];
    __shared__ float red[GPP][KS][M][16];
    uint16_t *xs = (uint16_t *)gsl;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 15u, g = lane >> 4;
    uint8_t *ring = gsl + (((size_t)M * K * 2u + 1023u) & ~(size_t)1023u) +
                    wv * (GS_R * 2048u);
    /* chunk = 128 bytes of each of 16 rows; row stride in bytes */
    const uint32_t KB = BF ? 2u * K : K;
    const uint32_t nch = KB >> 7, nkb = K >> 7;
    const uint32_t part = wv % KS, slot = wv / KS;
    const uint32_t c0 = part * nch / KS, c1 = (part + 1) * nch / KS, nc = c1 - c0;
    const uint32_t groups = (O + 15) / 16, passes = (groups + GPP - 1) / GPP;
    const uint16_t *xa = xs + (size_t)min(n, (uint32_t)M - 1u) * K + (BF ? 16u : 32u) * g;
    /* pass ps's row group of this wave: its rows and load offsets (a
     * partial last group re-reads row O-1, outputs discarded) */
    auto rows_of = [&](uint32_t ps) {
        return W + (size_t)(ps * GPP + slot) * 16u * KB;
    };
    auto offs_of = [&](uint32_t ps) {
        return ghip_cdma_offsets(lane, KB, min(15u, O - 1u - (ps * GPP + slot) * 16u));
    };
    /* NA chunks in flight: chunk t's two 16-byte pieces in register set
     * t % NA ((ra0, ra1), (rb0, rb1), (rc0, rc1)) and LDS slot t % NA */
    constexpr uint32_t NA = BF ? 3u : 2u;
    ghip_u32x4 ra0, ra1, rb0, rb1, rc0, rc1;
    /* the first NA chunks of a pass, always all loaded (chunk indices
     * clamped): a fixed count of loads in flight, in a fixed order */
    auto prefetch = [&](const uint8_t *rows, const ghip_cdma &d) {
        ghip_rl_load(rows, d, min(c0, nch - 1u), ra0, ra1);
        __builtin_amdgcn_sched_barrier(0);
        ghip_rl_load(rows, d, min(c0 + 1u, nch - 1u), rb0, rb1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NA == 3u) {
            ghip_rl_load(rows, d, min(c0 + 2u, nch - 1u), rc0, rc1);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    /* x into LDS without delaying the weight stream: x goes by direct DMA
     * (1 KB pieces dealt to the waves, lanes past x re-read its last vector
     * into the 1 KB-rounded x region) ahead of the first pass's 2 NA chunk
     * loads, so waiting until no more than those are in flight means this
     * wave's x pieces have landed */
    {
        const uint32_t nvec = (uint32_t)M * (K >> 3), nxc = (nvec + 63u) >> 6;
        for (uint32_t c = wv; c < nxc; c += GS_NW)
            ghip_dma16(X + (size_t)min(c * 64u + lane, nvec - 1u) * 8u, gsl + c * 1024u);
        const uint32_t grp0 = min(blockIdx.x * GPP + slot, groups - 1u);
        prefetch(W + (size_t)grp0 * 16u * KB,
               ghip_cdma_offsets(lane, KB, min(15u, O - 1u - grp0 * 16u)));
        GHIP_VMCNT(2 * NA);
    }
    /* a bare barrier: __syncthreads() would also wait for the chunk loads
     * (its workgroup-scope release waits for every load in flight) */
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const bool exact = !BF && exact_flag != nullptr && *exact_flag != 0u;
    for (uint32_t ps = blockIdx.x; ps < passes; ps += gridDim.x) {
        const uint32_t grp = ps * GPP + slot;
        const bool live = grp < groups;
        if (live) {
            /* a wave with no chunks (K < KS * 128) contributes zeros */
            const uint32_t row0 = grp * 16;
            const uint8_t *rows = rows_of(ps);
            const ghip_cdma d = offs_of(ps);
            const float *srow = BF ? nullptr : S + (size_t)(row0 >> 7) * nkb;
            if (ps != blockIdx.x) prefetch(rows, d);
            ghip_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            /* chunk t: its registers into LDS slot t % NA, the registers
             * refilled with chunk t + NA (REFILL), the chunk read back in
             * the MFMA layout with this lane's activations and the scale */
            auto step = [&](auto refill_c, uint32_t t, ghip_u32x4 &v0, ghip_u32x4 &v1,
                            uint8_t *buf) {
                ghip_rl_store(buf, lane, v0, v1);
                if constexpr (decltype(refill_c)::value) {
                    __builtin_amdgcn_sched_barrier(0);
                    ghip_rl_load(rows, d, c0 + t + NA, v0, v1);
                    __builtin_amdgcn_sched_barrier(0);
                }
                const uint32_t c = c0 + t;
                const ghip_chunk cw = ghip_cdma_read(buf, n, g);
                if constexpr (BF) {
                    const ghip_bf16x8 *a = (const ghip_bf16x8 *)(xa + c * 64u);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        a[0], __builtin_bit_cast(ghip_bf16x8, cw.lo), acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        a[1], __builtin_bit_cast(ghip_bf16x8, cw.hi), acc, 0, 0, 0);
                } else {
                    ghip_bf16x8 a4[4];
                    ghip_read_a4(xa + c * 128u, a4);
                    const float sc = ghip_sload(srow, c);
                    if (exact) ghip_chunk_mfma_a<true>(cw, sc, a4, acc);
                    else ghip_chunk_mfma_a<false>(cw, sc, a4, acc);
                }
            };
            using RF = std::true_type;
            using NR = std::false_type;
            uint32_t t = 0;
            if constexpr (NA == 2u) {
                for (; t + 3u < nc; t += 2) {
                    step(RF{}, t, ra0, ra1, ring);
                    step(RF{}, t + 1u, rb0, rb1, ring + 2048u);
                }
                if (nc - t == 3u) {
                    step(RF{}, t, ra0, ra1, ring);
                    step(NR{}, t + 1u, rb0, rb1, ring + 2048u);
                    step(NR{}, t + 2u, ra0, ra1, ring);
                } else if (nc - t == 2u) {
                    step(NR{}, t, ra0, ra1, ring);
                    step(NR{}, t + 1u, rb0, rb1, ring + 2048u);
                } else if (nc - t == 1u) {
                    step(NR{}, t, ra0, ra1, ring);
                }
            } else {
                for (; t + 5u < nc; t += 3) {
                    step(RF{}, t, ra0, ra1, ring);
                    step(RF{}, t + 1u, rb0, rb1, ring + 2048u);
                    step(RF{}, t + 2u, rc0, rc1, ring + 4096u);
                }
                const uint32_t rem = nc - t;
                if (rem == 5u) {
                    step(RF{}, t, ra0, ra1, ring);
                    step(RF{}, t + 1u, rb0, rb1, ring + 2048u);
                    step(NR{}, t + 2u, rc0, rc1, ring + 4096u);
                    step(NR{}, t + 3u, ra0, ra1, ring);
                    step(NR{}, t + 4u, rb0, rb1, ring + 2048u);
                } else if (rem == 4u) {
                    step(RF{}, t, ra0, ra1, ring);
                    step(NR{}, t + 1u, rb0, rb1, ring + 2048u);
                    step(NR{}, t + 2u, rc0, rc1, ring + 4096u);
                    step(NR{}, t + 3u, ra0, ra1, ring);
                } else {
                    if (rem > 0u) step(NR{}, t, ra0, ra1, ring);
                    if (rem > 1u) step(NR{}, t + 1u, rb0, rb1, ring + 2048u);
                    if (rem > 2u) step(NR{}, t + 2u, rc0, rc1, ring + 4096u);
                }
            }
            if (g == 0) {
#pragma unroll
                for (int i = 0; i < M; i++) red[slot][part][i][n] = acc[i];
            }
        } else {
            /* the pass's prefetched chunks are not used */
            GHIP_VMCNT(0);
        }
        __syncthreads();
        if (tid < GPP * M * 16u) {
            const uint32_t sl = tid / (M * 16u), rem = tid - sl * (M * 16u);
            const uint32_t m = rem >> 4, nn = rem & 15u;
            const uint32_t gp = ps * GPP + sl;
            if (gp < groups && gp * 16 + nn < O) {
                float s = 0.0f;
#pragma unroll
                for (int k = 0; k < KS; k++) s += red[sl][k][m][nn];
                Y[(size_t)m * O + gp * 16 + nn] = (uint16_t)ghip_bf16_bits(s);
            }
        }
        __syncthreads();
    }
}

static uint32_t g_gs_ncu;                 /* CUs: the streaming grid bound */

/* LDS the streaming GEMV needs for M token rows of length K */
static size_t gs_lds(size_t M, size_t K) {
    return ((M * K * 2 + 1023) & ~(size_t)1023) + (size_t)GS_NW * GS_R * 2048;
}

template <int M>
static hipError_t launch_gemv_m(const uint8_t *codes, const float *scales,
                                const uint16_t *x, uint16_t *y, size_t O,
                                size_t K, const uint32_t *exact_dev,
                                hipEvent_t ev0, hipEvent_t ev1, hipStream_t st) {
    const size_t groups = (O + 15) / 16;
    if (g_gs_ncu && gs_lds(M, K) <= GS_LDS) {
        const size_t lds = gs_lds(M, K);
        if ((groups + 3) / 4 >= g_gs_ncu) {          /* KS = 2: 4 groups a pass */
            uint32_t g = (uint32_t)((groups + 3) / 4);
            if (g > g_gs_ncu) g = g_gs_ncu;
            GHIP_LAUNCH(ev0, ev1, (k_fp8_gemv_stream<M, 2>), dim3(g), dim3(GS_NW * 64),
                        lds, st, codes, scales, x, y, (uint32_t)O, (uint32_t)K, exact_dev);
        } else {                                       /* KS = 8: 1 group a pass */
            uint32_t g = (uint32_t)groups;
            if (g > g_gs_ncu) g = g_gs_ncu;
            GHIP_LAUNCH(ev0, ev1, (k_fp8_gemv_stream<M, 8>), dim3(g), dim3(GS_NW * 64),
                        lds, st, codes, scales, x, y, (uint32_t)O, (uint32_t)K, exact_dev);
        }
        return hipGetLastError();
    }
    size_t lds = (size_t)M * K * 2;
    uint32_t nkb = (uint32_t)((K + 127) / 128);
    uint32_t g = (uint32_t)groups;
    GHIP_LAUNCH(ev0, ev1, k_fp8_gemv<M>, dim3(g), dim3(GEMV_NW * 64), lds, st,
                codes, scales, x, y, (uint32_t)O, (uint32_t)K, nkb, exact_dev);
    return hipGetLastError();
}

/* Rows of X from which the FP8 linear runs as one GEMM (below: GEMV passes
 * of <= 4 rows, each reading the weights once). */
#define GHIP_GEMM_MIN_M 16

/* Largest dynamic LDS the GEMV stages x into (per workgroup). */
#define GEMV_LDS_MAX (48u * 1024u)

extern "C" hipError_t ghip_launch_fp8_linear(const uint8_t *codes,
                                             const float *scales,
                                             const uint16_t *x, uint16_t *y,
                                             size_t M, size_t O, size_t K,
                                             const uint32_t *exact_dev,
                                             const hipEvent_t *ev,
                                             hipStream_t st) {
    if (M == 0 || O == 0) return hipSuccess;
    if (K == 0 || O > 0x7fffffffu || K > 0x7fffffffu || M > 0x7fffffffu)
        return hipErrorInvalidValue;
    /* timing events: start on the first launch, stop on the last */
    hipEvent_t ev0 = ev ? ev[0] : nullptr, ev1 = ev ? ev[1] : nullptr;
    bool fast = (K % 128 == 0) && (((uintptr_t)codes & 15) == 0)
             && (((uintptr_t)x & 15) == 0) && K * 2 <= GEMV_LDS_MAX;
    if (!fast) {
        uint32_t nkb = (uint32_t)((K + 127) / 128);
        size_t items = M * O;
        if (items > 0xffffffffull * 4) return hipErrorInvalidValue;
        GHIP_LAUNCH(ev0, ev1, k_fp8_linear_any, dim3((uint32_t)((items + 3) / 4)),
                    dim3(256), 0, st, codes, scales, x, y, (uint32_t)M,
                    (uint32_t)O, (uint32_t)K, nkb);
        return hipGetLastError();
    }
    /* from GHIP_GEMM_MIN_M rows on, the weights are read once by the MFMA
     * GEMM instead of once per group of <= 4 rows */
    if (M >= GHIP_GEMM_MIN_M && g_gs_ncu && ghip_fp8_gemm_fits(M, O, K, codes, x, y))
        return ghip_launch_fp8_gemm(codes, scales, x, y, M, O, K, exact_dev, g_gs_ncu, ev,
                                    st);
    /* m-groups of up to 4 rows, each as large as the x staging allows */
    size_t m0 = 0;
    while (m0 < M) {
        size_t mc = M - m0;
        if (mc > 4) mc = 4;
        while (mc > 1 && mc * K * 2 > GEMV_LDS_MAX) mc--;
        const uint16_t *xm = x + m0 * K;
        uint16_t *ym = y + m0 * O;
        hipEvent_t a = m0 == 0 ? ev0 : nullptr, b = m0 + mc == M ? ev1 : nullptr;
        hipError_t e;
        switch (mc) {
        case 4: e = launch_gemv_m<4>(codes, scales, xm, ym, O, K, exact_dev, a, b, st); break;
        case 3: e = launch_gemv_m<3>(codes, scales, xm, ym, O, K, exact_dev, a, b, st); break;
        case 2: e = launch_gemv_m<2>(codes, scales, xm, ym, O, K, exact_dev, a, b, st); break;
        default: e = launch_gemv_m<1>(codes, scales, xm, ym, O, K, exact_dev, a, b, st); break;
        }
        if (e != hipSuccess) return e;
        m0 += mc;
    }
    return hipSuccess;
}

template <int M>
static hipError_t launch_bf16_gemv_m(const uint16_t *w, const uint16_t *x, uint16_t *y,
                                     size_t O, size_t K, hipEvent_t ev0, hipEvent_t ev1,
                                     hipStream_t st) {
    const size_t groups = (O + 15) / 16;
    const size_t lds = gs_lds(M, K);
    const uint8_t *wb = (const uint8_t *)w;
    if ((groups + 3) / 4 >= g_gs_ncu) {              /* KS = 2: 4 groups a pass */
        uint32_t g = (uint32_t)((groups + 3) / 4);
        if (g > g_gs_ncu) g = g_gs_ncu;
        GHIP_LAUNCH(ev0, ev1, (k_fp8_gemv_stream<M, 2, true>), dim3(g), dim3(GS_NW * 64),
                    lds, st, wb, nullptr, x, y, (uint32_t)O, (uint32_t)K, nullptr);
    } else {                                           /* KS = 8: 1 group a pass */
        uint32_t g = (uint32_t)groups;
        if (g > g_gs_ncu) g = g_gs_ncu;
        GHIP_LAUNCH(ev0, ev1, (k_fp8_gemv_stream<M, 8, true>), dim3(g), dim3(GS_NW * 64),
                    lds, st, wb, nullptr, x, y, (uint32_t)O, (uint32_t)K, nullptr);
    }
    return hipGetLastError();
}

extern "C" hipError_t ghip_launch_bf16_linear(const uint16_t *w,
                                              const uint16_t *x, uint16_t *y,
                                              size_t M, size_t O, size_t K,
                                              const hipEvent_t *ev, hipStream_t st) {
    if (M == 0 || O == 0) return hipSuccess;
    if (K == 0 || O > 0x7fffffffu || K > 0x7fffffffu || M > 0x7fffffffu)
        return hipErrorInvalidValue;
    /* timing events: start on the first launch, stop on the last */
    hipEvent_t ev0 = ev ? ev[0] : nullptr, ev1 = ev ? ev[1] : nullptr;
    /* the streaming MFMA GEMV, in groups of <= 4 token rows (each reading
     * the weights once), when the shape and alignment allow */
    if (g_gs_ncu && K % 64 == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0
        && gs_lds(1, K) <= GS_LDS) {
        size_t m0 = 0;
        while (m0 < M) {
            size_t mc = M - m0;
            if (mc > 4) mc = 4;
            while (mc > 1 && gs_lds(mc, K) > GS_LDS) mc--;
            const uint16_t *xm = x + m0 * K;
            uint16_t *ym = y + m0 * O;
            hipEvent_t a = m0 == 0 ? ev0 : nullptr, b = m0 + mc == M ? ev1 : nullptr;
            hipError_t e;
            switch (mc) {
            case 4: e = launch_bf16_gemv_m<4>(w, xm, ym, O, K, a, b, st); break;
            case 3: e = launch_bf16_gemv_m<3>(w, xm, ym, O, K, a, b, st); break;
            case 2: e = launch_bf16_gemv_m<2>(w, xm, ym, O, K, a, b, st); break;
            default: e = launch_bf16_gemv_m<1>(w, xm, ym, O, K, a, b, st); break;
            }
            if (e != hipSuccess) return e;
            m0 += mc;
        }
        return hipSuccess;
    }
    size_t items = M * O;
    if (items > 0xffffffffull * 4) return hipErrorInvalidValue;
    GHIP_LAUNCH(ev0, ev1, k_bf16_linear_any, dim3((uint32_t)((items + 3) / 4)),
                dim3(256), 0, st, w, x, y, (uint32_t)M, (uint32_t)O, (uint32_t)K);
    return hipGetLastError();
}

template <int M>
static hipError_t gs_attr(void) {
    const void *ks[4] = {(const void *)k_fp8_gemv_stream<M, 2>,
                         (const void *)k_fp8_gemv_stream<M, 8>,
                         (const void *)k_fp8_gemv_stream<M, 2, true>,
                         (const void *)k_fp8_gemv_stream<M, 8, true>};
    for (int i = 0; i < 4; i++) {
        hipError_t e = hipFuncSetAttribute(ks[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                           GS_LDS);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

extern "C" hipError_t ghip_linear_init(uint32_t n_cu) {
    hipError_t e;
    if ((e = gs_attr<1>()) != hipSuccess || (e = gs_attr<2>()) != hipSuccess
        || (e = gs_attr<3>()) != hipSuccess || (e = gs_attr<4>()) != hipSuccess)
        return e;
    g_gs_ncu = n_cu;
    return hipSuccess;
}
