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

/* numpy-stable sigmoid (c/gmhc.h:157-160) with the device expf. */
__device__ __forceinline__ float ghip_sigmoid_np(float x) {
    float e = expf(-fabsf(x));
    return x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
}

/* SwiGLU on bf16-valued g and u (c/gmoe.h:217-225): gate clamped above,
 * up clamped both sides, h = bf16(bf16(g * sigmoid(g)) * u). */
__device__ __forceinline__ uint32_t ghip_swiglu(float g, float u, float limit) {
    if (g > limit) g = limit;
    if (u > limit) u = limit;
    else if (u < -limit) u = -limit;
    float hv = ghip_bf16_round(g * ghip_sigmoid_np(g));
    return ghip_bf16_bits(hv * u);
}

#endif /* GHIP_DEVICE_H */
