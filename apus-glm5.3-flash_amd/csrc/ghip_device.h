/*
 * ghip_device.h — device-side numerics shared by the gfx950 kernels.
 *
 * Numerics contract restated from the reference (c/num.h:136-166,
 * c/fp8blk.h:6-33):
 *   e4m3(c)  exact: e != 0 -> (8+m)*2^(e-10), e == 0 -> m*2^-9, sign bit 7;
 *            the two NaN codes 0x7F/0xFF decode as +-480.
 *   deq      bf16_rne(e4m3(code) * scale): ONE fp32 multiply, then the RNE
 *            narrow (u += 0x7FFF + ((u >> 16) & 1), NaN passes through).
 *
 * Two decode paths, both producing the reference bits on finite codes:
 *   - FAST: v_cvt_pk_f32_fp8 (gfx950 decodes OCP E4M3FN) + v_mul_f32 +
 *     v_cvt_pk_bf16_f32 (RNE). Used for weights with no NaN code; the GPU
 *     gate (tests/test_gpu_dequant.py) checks it on every finite code x
 *     scale corners, including subnormal products.
 *   - EXACT: integer decode (NaN codes -> +-480, as the reference) and the
 *     integer RNE narrow. Used when a matrix holds a 0x7F/0xFF code.
 */
#ifndef GHIP_DEVICE_H
#define GHIP_DEVICE_H

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

typedef __bf16 ghip_bf16x8 __attribute__((ext_vector_type(8)));
typedef float ghip_f32x4 __attribute__((ext_vector_type(4)));
typedef float ghip_f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int ghip_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float ghip_bf16_f32(uint32_t b) {
    return __uint_as_float(b << 16);
}

/* c/num.h:153-159 RNE narrow, integer form (NaN passes through). */
__device__ __forceinline__ uint32_t ghip_bf16_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u >> 16;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

/* c/num.h:143-151: the same rounding kept in an fp32 container. */
__device__ __forceinline__ float ghip_bf16_round(float x) {
    return __uint_as_float(ghip_bf16_bits(x) << 16);
}

/* c/num.h:136-141, integer construction: normal codes have exponent field
 * e + 120 and mantissa m << 20; subnormal codes are m * 2^-9 (exact). */
__device__ __forceinline__ float ghip_e4m3_exact(uint32_t c) {
    uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20))
                : (float)m * 0x1p-9f;
    return (c & 0x80u) ? -v : v;
}

typedef unsigned int ghip_u32x2 __attribute__((ext_vector_type(2)));

/* Four codes of one dword -> four dequantized bf16 packed in two dwords
 * (element j in bits [16*(j&1), +16) of dword j/2). */
template <bool EXACT>
__device__ __forceinline__ ghip_u32x2 ghip_deq4(uint32_t d, float s) {
    ghip_u32x2 r;
    if (EXACT) {
        uint32_t b0 = ghip_bf16_bits(ghip_e4m3_exact(d & 0xffu) * s);
        uint32_t b1 = ghip_bf16_bits(ghip_e4m3_exact((d >> 8) & 0xffu) * s);
        uint32_t b2 = ghip_bf16_bits(ghip_e4m3_exact((d >> 16) & 0xffu) * s);
        uint32_t b3 = ghip_bf16_bits(ghip_e4m3_exact(d >> 24) * s);
        r[0] = b0 | (b1 << 16);
        r[1] = b2 | (b3 << 16);
    } else {
        ghip_f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false);
        ghip_f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
        typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
        bf2 p, q;
        p[0] = (__bf16)(a[0] * s);
        p[1] = (__bf16)(a[1] * s);
        q[0] = (__bf16)(b[0] * s);
        q[1] = (__bf16)(b[1] * s);
        r[0] = __builtin_bit_cast(uint32_t, p);
        r[1] = __builtin_bit_cast(uint32_t, q);
    }
    return r;
}

/* 16 codes (one 16-byte load) -> 8 dwords of packed bf16: lo holds codes
 * 0..7, hi codes 8..15. */
template <bool EXACT>
__device__ __forceinline__ void ghip_deq16_u32(ghip_u32x4 c, float s,
                                               ghip_u32x4 &lo, ghip_u32x4 &hi) {
    ghip_u32x2 a = ghip_deq4<EXACT>(c[0], s), b = ghip_deq4<EXACT>(c[1], s);
    ghip_u32x2 e = ghip_deq4<EXACT>(c[2], s), f = ghip_deq4<EXACT>(c[3], s);
    lo = (ghip_u32x4){a[0], a[1], b[0], b[1]};
    hi = (ghip_u32x4){e[0], e[1], f[0], f[1]};
}

/* 16 codes -> two MFMA bf16x8 operands (codes 0..7, codes 8..15). */
template <bool EXACT>
__device__ __forceinline__ void ghip_deq16(ghip_u32x4 c, float s,
                                           ghip_bf16x8 &b0, ghip_bf16x8 &b1) {
    ghip_u32x4 lo, hi;
    ghip_deq16_u32<EXACT>(c, s, lo, hi);
    b0 = __builtin_bit_cast(ghip_bf16x8, lo);
    b1 = __builtin_bit_cast(ghip_bf16x8, hi);
}

/* ---- 16-row GEMV chunk (the streaming unit of every GEMV kernel) --------
 * A wave owns 16 output rows; a chunk is one 128-wide k block of each row
 * (one F32 scale). Lane l = 16*g + n holds row n, codes [32g, 32g+32) of
 * the chunk: two 16-byte loads, so one wave covers 16 full 128-byte lines.
 * The 32 codes dequantize to four bf16x8 MFMA B operands; MFMA i uses codes
 * [8i, 8i+8) of every lane group, i.e. k-slot (g, j) <-> k = 32g + 8i + j,
 * and the A operand (activation, from LDS) is read with the same mapping,
 * so each v_mfma_f32_16x16x32_bf16 sums a permutation of 32 exact
 * products. */
struct ghip_chunk {
    ghip_u32x4 lo, hi;
};

__device__ __forceinline__ ghip_chunk ghip_chunk_load(const uint8_t *p) {
    ghip_chunk c;
    c.lo = __builtin_nontemporal_load((const ghip_u32x4 *)p);
    c.hi = __builtin_nontemporal_load((const ghip_u32x4 *)(p + 16));
    return c;
}

/* acc += A(xa[0..32)) . B(dequant(chunk)); xa points at this lane's 32
 * activations of the chunk (row m of x, k = 128c + 32g). */
template <bool EXACT>
__device__ __forceinline__ void ghip_chunk_mfma(const ghip_chunk &c, float sc,
                                                const uint16_t *xa,
                                                ghip_f32x4 &acc) {
    ghip_bf16x8 b0, b1, b2, b3;
    ghip_deq16<EXACT>(c.lo, sc, b0, b1);
    ghip_deq16<EXACT>(c.hi, sc, b2, b3);
    const ghip_bf16x8 *a = (const ghip_bf16x8 *)xa;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b1, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b2, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[3], b3, acc, 0, 0, 0);
}

/* the same with this lane's four activation operands already in registers
 * (read from LDS together with the chunk's codes, so one LDS wait covers
 * both) */
template <bool EXACT>
__device__ __forceinline__ void ghip_chunk_mfma_a(const ghip_chunk &c, float sc,
                                                  const ghip_bf16x8 (&a)[4],
                                                  ghip_f32x4 &acc) {
    ghip_bf16x8 b0, b1, b2, b3;
    ghip_deq16<EXACT>(c.lo, sc, b0, b1);
    ghip_deq16<EXACT>(c.hi, sc, b2, b3);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b1, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b2, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[3], b3, acc, 0, 0, 0);
}

__device__ __forceinline__ void ghip_read_a4(const uint16_t *xa, ghip_bf16x8 (&a)[4]) {
    const ghip_bf16x8 *p = (const ghip_bf16x8 *)xa;
    a[0] = p[0];
    a[1] = p[1];
    a[2] = p[2];
    a[3] = p[3];
}

/* ---- activation staging without serializing the weight stream ----------
 * vmcnt retires loads in issue order, so an activation load issued AFTER
 * the weight loads makes its LDS write wait for every weight byte. Stage in
 * two steps instead: ghip_stage_load (before the weight loads) pulls up to
 * GHIP_STAGE_V 16-byte vectors per thread into registers; ghip_stage_store
 * (after them) writes them to LDS, waiting only for the activation loads.
 * Any remainder (larger activations) is copied directly. nvec >= 1. */
#define GHIP_STAGE_V 4

struct ghip_stage {
    ghip_u32x4 v[GHIP_STAGE_V];
};

__device__ __forceinline__ void ghip_stage_load(ghip_stage &st, const uint16_t *src,
                                                uint32_t nvec, uint32_t tid,
                                                uint32_t nthr) {
    /* unconditional loads (index clamped, extra values unused): straight-line
     * code lets the compiler wait for these with vmcnt(#weight loads) */
#pragma unroll
    for (int j = 0; j < GHIP_STAGE_V; j++) {
        uint32_t i = min(tid + j * nthr, nvec - 1u);
        st.v[j] = *(const ghip_u32x4 *)(src + ((size_t)i << 3));
    }
}

__device__ __forceinline__ void ghip_stage_store(const ghip_stage &st, uint16_t *dst,
                                                 const uint16_t *src, uint32_t nvec,
                                                 uint32_t tid, uint32_t nthr) {
    /* unconditional too (a clamped index rewrites element nvec-1 with its
     * own value): a conditional store lets the compiler sink the load into
     * the branch, behind the weight loads */
#pragma unroll
    for (int j = 0; j < GHIP_STAGE_V; j++) {
        uint32_t i = min(tid + j * nthr, nvec - 1u);
        *(ghip_u32x4 *)(dst + ((size_t)i << 3)) = st.v[j];
    }
    for (uint32_t i = tid + GHIP_STAGE_V * nthr; i < nvec; i += nthr)
        *(ghip_u32x4 *)(dst + ((size_t)i << 3)) = *(const ghip_u32x4 *)(src + ((size_t)i << 3));
}

/* ---- wave-local activation staging -------------------------------------
 * A wave that owns chunks c = w, w + step, ... of a row stages only those
 * 128-wide slices of the activation rows (M rows, row stride K elements)
 * into LDS (same [M][K] layout), and only its own lanes read them back: no
 * workgroup barrier, and 1/step of the activation traffic per wave. Vector
 * v (16 bytes) of the wave's list = (chunk u, row m, part p) with
 * v = (u*M + m)*16 + p. Up to GHIP_STAGE_V vectors per lane go through
 * registers (loaded before the weights, see ghip_stage_load); the rest is
 * copied directly. */
__device__ __forceinline__ size_t ghip_wst_off(uint32_t v, uint32_t M, uint32_t K,
                                               uint32_t w, uint32_t step) {
    const uint32_t p = v & 15u, um = v >> 4, u = um / M, m = um - u * M;
    return (size_t)m * K + (size_t)(w + u * step) * 128u + p * 8u;
}

__device__ __forceinline__ void ghip_wstage_load(ghip_stage &st, const uint16_t *src,
                                                 uint32_t M, uint32_t K, uint32_t nch,
                                                 uint32_t w, uint32_t step,
                                                 uint32_t lane) {
    const uint32_t nwch = w < nch ? (nch - w + step - 1) / step : 0u;
    const uint32_t nv = nwch * M * 16u;
#pragma unroll
    for (int j = 0; j < GHIP_STAGE_V; j++) {
        uint32_t v = min(lane + 64u * j, nv ? nv - 1u : 0u);
        st.v[j] = *(const ghip_u32x4 *)(src + ghip_wst_off(v, M, K, w, step));
    }
}

__device__ __forceinline__ void ghip_wstage_store(const ghip_stage &st, uint16_t *dst,
                                                  const uint16_t *src, uint32_t M,
                                                  uint32_t K, uint32_t nch, uint32_t w,
                                                  uint32_t step, uint32_t lane) {
    const uint32_t nwch = w < nch ? (nch - w + step - 1) / step : 0u;
    const uint32_t nv = nwch * M * 16u;
#pragma unroll
    for (int j = 0; j < GHIP_STAGE_V; j++) {
        uint32_t v = min(lane + 64u * j, nv ? nv - 1u : 0u);
        *(ghip_u32x4 *)(dst + ghip_wst_off(v, M, K, w, step)) = st.v[j];
    }
    for (uint32_t v = lane + 64u * GHIP_STAGE_V; v < nv; v += 64u)
        *(ghip_u32x4 *)(dst + ghip_wst_off(v, M, K, w, step)) =
            *(const ghip_u32x4 *)(src + ghip_wst_off(v, M, K, w, step));
    /* the wave's own LDS writes complete before its lanes read them */
    __builtin_amdgcn_s_waitcnt(0xc07f);           /* lgkmcnt(0) */
    __builtin_amdgcn_wave_barrier();
}

/* Direct wave-local copy of nvec 16-byte vectors (no register staging). */
__device__ __forceinline__ void ghip_wcopy(uint16_t *dst, const uint16_t *src,
                                           uint32_t nvec, uint32_t lane) {
    for (uint32_t v = lane; v < nvec; v += 64u)
        *(ghip_u32x4 *)(dst + ((size_t)v << 3)) = *(const ghip_u32x4 *)(src + ((size_t)v << 3));
    __builtin_amdgcn_s_waitcnt(0xc07f);           /* lgkmcnt(0) */
    __builtin_amdgcn_wave_barrier();
}

/* ---- direct global -> LDS loads (gfx950 global_load_lds_dwordx4) -------
 * Lane l of the wave writes its 16 bytes to lds_wave + 16*l, bypassing
 * registers; completion is tracked by vmcnt like any vector load. */
typedef __attribute__((address_space(3))) void ghip_lds_t;
typedef __attribute__((address_space(1))) void ghip_glb_t;
__device__ __forceinline__ void ghip_dma16(const void *src, void *lds_wave) {
    __builtin_amdgcn_global_load_lds((ghip_glb_t *)src, (ghip_lds_t *)lds_wave, 16, 0, 0);
}

/* s_waitcnt vmcnt(N), other counters untouched. */
#define GHIP_VMCNT(N) __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | 0x0F70)

/* vmcnt(LPS * min(m, M)): wait until at most min(m, M) stages of LPS loads
 * each are still in flight (m wave-uniform). */
template <uint32_t LPS, uint32_t M>
__device__ __forceinline__ void ghip_wait_stages(uint32_t m) {
    if constexpr (M == 0) {
        GHIP_VMCNT(0);
    } else {
        if (m >= M) GHIP_VMCNT(LPS * M);
        else ghip_wait_stages<LPS, M - 1>(m);
    }
}

/* Wave-uniform reads through the constant address space: scalar loads
 * (lgkmcnt), so they never wait behind a stream of vector loads. The data
 * must not change while the kernel runs. */
__device__ __forceinline__ float ghip_sload(const float *p, uint32_t i) {
    return ((const __attribute__((address_space(4))) float *)p)[i];
}
__device__ __forceinline__ uint32_t ghip_sload_u32(const uint32_t *p, uint32_t i) {
    return ((const __attribute__((address_space(4))) uint32_t *)p)[i];
}

/* ---- streaming 16-row GEMV chunks through LDS ---------------------------
 * A chunk (16 weight rows x 128 codes = 2 KB, one scale block) lives in
 * LDS as [16 rows][8 pieces of 16 B] with piece p of row r at
 * (p ^ ((r >> 1) & 7)), so the MFMA-layout reads (lane 16g + n: row n,
 * pieces 2g and 2g+1) hit distinct banks. Two DMA instructions fill it:
 * instruction i, lane l -> row 8i + l/8, stored slot l % 8. */
struct ghip_cdma {
    uint32_t off0, off1;          /* global byte offsets (row * K + piece) */
};

/* rmax: rows past it (a partial last group) re-read row rmax */
__device__ __forceinline__ ghip_cdma ghip_cdma_offsets(uint32_t lane, uint32_t K,
                                                       uint32_t rmax = 15u) {
    ghip_cdma d;
    const uint32_t r0 = min(lane >> 3, rmax), r1 = min(8u + (lane >> 3), rmax);
    d.off0 = r0 * K + 16u * ((lane & 7u) ^ ((r0 >> 1) & 7u));
    d.off1 = r1 * K + 16u * ((lane & 7u) ^ ((r1 >> 1) & 7u));
    return d;
}

/* chunk c of the 16 rows at `rows` (row stride K) -> LDS chunk buffer */
__device__ __forceinline__ void ghip_cdma_issue(const uint8_t *rows, uint32_t c,
                                               const ghip_cdma &d, uint8_t *buf) {
    ghip_dma16(rows + (size_t)c * 128u + d.off0, buf);
    ghip_dma16(rows + (size_t)c * 128u + d.off1, buf + 1024);
}

/* ---- streaming chunks through registers ---------------------------------
 * The same whole-line pattern as the DMA (ghip_cdma_offsets: load i, lane
 * l -> row 8i + l/8, swizzled piece l % 8), as two 16-byte register loads
 * per lane; ghip_rl_store then writes them where the DMA would (lane l's
 * bytes at 16 l of each 1 KB half), so ghip_cdma_read reads either. Plain
 * register loads stream faster than global_load_lds on this part at the
 * same bytes in flight, and the compiler tracks their waits exactly. */
__device__ __forceinline__ void ghip_rl_load(const uint8_t *rows, const ghip_cdma &d,
                                             uint32_t c, ghip_u32x4 &v0, ghip_u32x4 &v1) {
    const uint8_t *p = rows + (size_t)c * 128u;
    v0 = __builtin_nontemporal_load((const ghip_u32x4 *)(p + d.off0));
    v1 = __builtin_nontemporal_load((const ghip_u32x4 *)(p + d.off1));
}

__device__ __forceinline__ void ghip_rl_store(uint8_t *buf, uint32_t lane, const ghip_u32x4 &v0,
                                              const ghip_u32x4 &v1) {
    *(ghip_u32x4 *)(buf + lane * 16u) = v0;
    *(ghip_u32x4 *)(buf + 1024u + lane * 16u) = v1;
}

/* this lane's 32 codes of a chunk in LDS (row n, pieces 2g, 2g+1) */
__device__ __forceinline__ ghip_chunk ghip_cdma_read(const uint8_t *buf, uint32_t n,
                                                    uint32_t g) {
    const uint32_t sw = (n >> 1) & 7u;
    ghip_chunk c;
    c.lo = *(const ghip_u32x4 *)(buf + n * 128u + 16u * ((2u * g) ^ sw));
    c.hi = *(const ghip_u32x4 *)(buf + n * 128u + 16u * ((2u * g + 1u) ^ sw));
    return c;
}

/* numpy-stable sigmoid (c/gmhc.h:157-160) with the device expf. */
__device__ __forceinline__ float ghip_sigmoid_np(float x) {
    float e = expf(-fabsf(x));
    return x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
}

/* SwiGLU on bf16-valued g and u (c/gmoe.h:217-225): gate clamped above,
 * up clamped both sides, h = bf16(bf16(g * sigmoid(g)) * u). */
__device__ __forceinline__ uint32_t ghip_swiglu(float g, float u, float limit) {
    g = g > limit ? limit : g;                   /* selects: no exec branches */
    u = u > limit ? limit : (u < -limit ? -limit : u);
    float hv = ghip_bf16_round(g * ghip_sigmoid_np(g));
    return ghip_bf16_bits(hv * u);
}

/* Launch with optional start/stop timing events carried by the dispatch
 * packet itself (hipExtLaunchKernelGGL): no extra marker packets between
 * launches, so the measured span is the kernel's own. */
#define GHIP_LAUNCH(ev0, ev1, kern, grid, block, lds, st, ...)                  \
    do {                                                                       \
        if ((ev0) || (ev1))                                                    \
            hipExtLaunchKernelGGL(kern, grid, block, lds, st, ev0, ev1, 0,     \
                                  __VA_ARGS__);                                \
        else                                                                   \
            hipLaunchKernelGGL(kern, grid, block, lds, st, __VA_ARGS__);       \
    } while (0)

#endif /* GHIP_DEVICE_H */
