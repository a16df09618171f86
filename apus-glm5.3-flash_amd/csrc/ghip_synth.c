/*
 * ghip_synth.c — deterministic synthetic inputs for the FP8-block MoE path
 * (C11, host side). One generator spec shared by the GPU path (bench.py,
 * the device fill kernels in k_synth.hip) and the CPU checker (tests/), so
 * both sides see identical bytes.
 *
 * Counter-based splitmix64: draw i of stream s under seed is
 *     key  = mix64(seed + (s + 1) * 0x632BE59BD9B4E019)
 *     u64  = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)
 * so any sub-range (a row, one expert of a bank) can be generated alone and
 * the device kernels reproduce the host bytes exactly (integer-only).
 *
 * Distributions:
 *   FP8 codes   uniform over the 254 finite E4M3 codes (0x7F/0xFF excluded):
 *               r = u64 % 254, code = r < 127 ? r : r + 1.
 *   scales      log-uniform in [lo, hi]: exp(ln lo + U * (ln hi - ln lo)),
 *               U = (u64 >> 11) * 2^-53, computed in double, host only.
 *   bf16 N(0,1) a 65536-entry quantile table T[i] = bf16(Phi^-1((i+.5)/2^16))
 *               indexed by the top 16 bits of u64 (integer-only on device).
 *   f32 N(0,1)  Box-Muller in double over draws 2i, 2i+1 (logits, host only).
 *   routing     uniform or Zipf(s) top-k with distinct experts per token;
 *               Zipf ranks map to expert ids through a seeded permutation;
 *               weights = softmax over k iid N(0,1) slot logits.
 */
#include "apus_synth.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

uint64_t apus_synth_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t apus_synth_key(uint64_t seed, uint64_t stream) {
    return apus_synth_mix64(seed + (stream + 1) * 0x632BE59BD9B4E019ull);
}

uint64_t apus_synth_u64(uint64_t key, uint64_t i) {
    return apus_synth_mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

static double synth_unit(uint64_t r) {            /* [0, 1) */
    return (double)(r >> 11) * 0x1p-53;
}

static uint16_t synth_bf16_bits(float x) {        /* RNE narrow */
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(u >> 16);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void apus_synth_fp8_codes(uint8_t *out, size_t n, uint64_t seed,
                          uint64_t stream, uint64_t offset) {
    uint64_t key = apus_synth_key(seed, stream);
    for (size_t i = 0; i < n; i++) {
        uint32_t r = (uint32_t)(apus_synth_u64(key, offset + i) % 254u);
        out[i] = (uint8_t)(r < 127u ? r : r + 1u);
    }
}

void apus_synth_scales(float *out, size_t n, uint64_t seed, uint64_t stream,
                       float lo, float hi) {
    uint64_t key = apus_synth_key(seed, stream);
    double a = log((double)lo), b = log((double)hi);
    for (size_t i = 0; i < n; i++)
        out[i] = (float)exp(a + synth_unit(apus_synth_u64(key, i)) * (b - a));
}

/* Inverse standard normal CDF: Acklam's rational approximation (relative
 * error < 1.2e-9) refined by one Halley step on erfc, which brings it to
 * double precision — far below the bf16 quantum the table is rounded to. */
static double synth_norm_ppf(double p) {
    static const double a[] = { -3.969683028665376e+01, 2.209460984245205e+02,
        -2.759285104469687e+02, 1.383577518672690e+02,
        -3.066479806614716e+01, 2.506628277459239e+00 };
    static const double b[] = { -5.447609879822406e+01, 1.615858368580409e+02,
        -1.556989798598866e+02, 6.680131188771972e+01,
        -1.328068155288572e+01 };
    static const double c[] = { -7.784894002430293e-03, -3.223964580411365e-01,
        -2.400758277161838e+00, -2.549732539343734e+00,
        4.374664141464968e+00, 2.938163982698783e+00 };
    static const double d[] = { 7.784695709041462e-03, 3.224671290700398e-01,
        2.445134137142996e+00, 3.754408661907416e+00 };
    const double plow = 0.02425, phigh = 1.0 - plow;
    double x;
    if (p < plow) {
        double q = sqrt(-2.0 * log(p));
        x = (((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5])
          / ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1.0);
    } else if (p <= phigh) {
        double q = p - 0.5, r = q * q;
        x = (((((a[0] * r + a[1]) * r + a[2]) * r + a[3]) * r + a[4]) * r + a[5]) * q
          / (((((b[0] * r + b[1]) * r + b[2]) * r + b[3]) * r + b[4]) * r + 1.0);
    } else {
        double q = sqrt(-2.0 * log(1.0 - p));
        x = -(((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5])
          / ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1.0);
    }
    double e = 0.5 * erfc(-x / sqrt(2.0)) - p;
    double u = e * sqrt(2.0 * M_PI) * exp(x * x / 2.0);
    return x - u / (1.0 + x * u / 2.0);
}

void apus_synth_normal_table(uint16_t *tab) {
    for (int i = 0; i < 65536; i++)
        tab[i] = synth_bf16_bits((float)synth_norm_ppf(((double)i + 0.5)
                                                       / 65536.0));
}

static uint16_t synth_tab[65536];
static int synth_tab_ready;

const uint16_t *apus_synth_normal_table_ptr(void) {
    if (!synth_tab_ready) {
        apus_synth_normal_table(synth_tab);
        synth_tab_ready = 1;
    }
    return synth_tab;
}

void apus_synth_bf16_normal(uint16_t *out, size_t n, uint64_t seed,
                            uint64_t stream, uint64_t offset) {
    const uint16_t *tab = apus_synth_normal_table_ptr();
    uint64_t key = apus_synth_key(seed, stream);
    for (size_t i = 0; i < n; i++)
        out[i] = tab[apus_synth_u64(key, offset + i) >> 48];
}

void apus_synth_f32_normal(float *out, size_t n, uint64_t seed,
                           uint64_t stream, uint64_t offset) {
    uint64_t key = apus_synth_key(seed, stream);
    for (size_t i = 0; i < n; i++) {
        uint64_t j = 2 * (offset + i);
        double u1 = ((double)(apus_synth_u64(key, j) >> 11) + 1.0) * 0x1p-53;
        double u2 = synth_unit(apus_synth_u64(key, j + 1));
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2));
    }
}

/* Softmax over k slot logits: m = max, e_j = expf(l_j - m), s = sum in
 * ascending j, w_j = e_j / s. */
static void synth_softmax(const float *l, int k, float *w) {
    float m = l[0];
    for (int j = 1; j < k; j++) if (l[j] > m) m = l[j];
    float s = 0.0f;
    for (int j = 0; j < k; j++) { w[j] = expf(l[j] - m); s = s + w[j]; }
    for (int j = 0; j < k; j++) w[j] = w[j] / s;
}

int apus_synth_route(int32_t *idx, float *w, size_t T, int E, int k,
                     double zipf_s, uint64_t seed) {
    if (k <= 0 || k > E || E <= 0) return 1;
    double *cdf = (double *)malloc((size_t)E * sizeof(double));
    int32_t *perm = (int32_t *)malloc((size_t)E * sizeof(int32_t));
    float *l = (float *)malloc((size_t)k * sizeof(float));
    if (!cdf || !perm || !l) { free(cdf); free(perm); free(l); return 1; }
    /* rank -> expert permutation (Fisher-Yates, stream 1) */
    uint64_t pk = apus_synth_key(seed, 1);
    for (int e = 0; e < E; e++) perm[e] = e;
    for (int e = E - 1; e > 0; e--) {
        int j = (int)(apus_synth_u64(pk, (uint64_t)e) % (uint64_t)(e + 1));
        int32_t t = perm[e]; perm[e] = perm[j]; perm[j] = t;
    }
    double acc = 0.0;
    for (int r = 0; r < E; r++) {
        acc += zipf_s > 0.0 ? pow((double)(r + 1), -zipf_s) : 1.0;
        cdf[r] = acc;
    }
    uint64_t dk = apus_synth_key(seed, 2);
    uint64_t draw = 0;
    for (size_t t = 0; t < T; t++) {
        int32_t *it = idx + t * (size_t)k;
        int got = 0;
        while (got < k) {
            double u = synth_unit(apus_synth_u64(dk, draw++)) * acc;
            int lo = 0, hi = E - 1;                  /* first cdf > u */
            while (lo < hi) {
                int mid = (lo + hi) / 2;
                if (cdf[mid] > u) hi = mid; else lo = mid + 1;
            }
            int32_t e = perm[lo];
            int dup = 0;
            for (int q = 0; q < got; q++) if (it[q] == e) { dup = 1; break; }
            if (!dup) it[got++] = e;
        }
        apus_synth_f32_normal(l, (size_t)k, seed, 3, (uint64_t)t * (uint64_t)k);
        synth_softmax(l, k, w + t * (size_t)k);
    }
    free(cdf); free(perm); free(l);
    return 0;
}

/* Expert bank stream ids: bank b, expert e, member j in
 * {gate codes, gate scales, up codes, up scales, down codes, down scales}. */
uint64_t apus_synth_expert_stream(int bank, int expert, int member) {
    return ((uint64_t)bank * 65536ull + (uint64_t)expert) * 8ull
         + (uint64_t)member + 1024ull;
}
