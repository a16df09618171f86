/*
 * oracle/apus_oracle.c — TEST INFRASTRUCTURE ONLY (the parity checker and the
 * timed CPU baseline). A clean-room C restatement of the apus reference CPU
 * semantics for the FP8-block MoE hot path; see apus_oracle.h for the
 * function list and the reference file:line each one follows.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -mavx2 -mf16c). Contraction
 * is pinned off: the anchors are two-rounding mul+add sequences.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library. The product library never links it.
 */
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "apus_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define APO_X86 1
#else
#define APO_X86 0
#endif

/* ======================================================================== */
/* codec                                                                     */
/* ======================================================================== */

/* c/num.h:136-141. OCP E4M3 decode, exact: e != 0 -> (8+m)*2^(e-10),
 * e == 0 -> m*2^-9; sign bit 7. The two NaN codes (0x7F/0xFF) decode as
 * +-480 (e=15, m=7 read as a normal), as the reference does. */
float apo_e4m3_f32(uint8_t c) {
    int e = (c >> 3) & 15, m = c & 7;
    float v = e ? ldexpf((float)(8 + m), e - 10) : ldexpf((float)m, -9);
    return (c & 0x80) ? -v : v;
}

/* c/num.h:153-159. fp32 -> bf16 code, round-to-nearest-even on the low 16
 * bits; NaN passes through as its high half. */
uint16_t apo_bf16_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(u >> 16);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* c/num.h:143-151. Same rounding, result kept in an fp32 container. */
float apo_bf16_round(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&x, &u, 4);
    return x;
}

/* c/num.h:161-166. Exact widen. */
float apo_bf16_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* c/fp8blk.h:109-111 */
size_t apo_nblocks(size_t n) { return (n + 127) / 128; }

/* ======================================================================== */
/* persistent row-partition pool (c/pool.h:144-185 semantics: [0,n) split    */
/* into contiguous blocks, lane 0 = caller; every output row is computed by  */
/* one lane with the per-row code, so results do not depend on the count)    */
/* ======================================================================== */

#define APO_MAX_THREADS 64

typedef void (*apo_rows_fn)(void *ctx, size_t r0, size_t r1);

static struct {
    pthread_mutex_t mu;
    pthread_cond_t work, done;
    pthread_t tid[APO_MAX_THREADS];
    int spawned;                 /* worker threads alive (lanes 1..spawned) */
    uint64_t gen;
    int nlane, pending;
    apo_rows_fn fn;
    void *ctx;
    size_t lo[APO_MAX_THREADS], hi[APO_MAX_THREADS];
} apo_pool = { .mu = PTHREAD_MUTEX_INITIALIZER,
               .work = PTHREAD_COND_INITIALIZER,
               .done = PTHREAD_COND_INITIALIZER };
static pthread_mutex_t apo_pool_call_mu = PTHREAD_MUTEX_INITIALIZER;

int apo_default_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > APO_MAX_THREADS) n = APO_MAX_THREADS;
    return (int)n;
}

static void *apo_worker(void *arg) {
    int lane = (int)(intptr_t)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&apo_pool.mu);
    for (;;) {
        while (apo_pool.gen == seen)
            pthread_cond_wait(&apo_pool.work, &apo_pool.mu);
        seen = apo_pool.gen;
        int active = lane < apo_pool.nlane;
        apo_rows_fn fn = apo_pool.fn;
        void *ctx = apo_pool.ctx;
        size_t lo = apo_pool.lo[lane], hi = apo_pool.hi[lane];
        pthread_mutex_unlock(&apo_pool.mu);
        if (active && hi > lo) fn(ctx, lo, hi);
        pthread_mutex_lock(&apo_pool.mu);
        if (active && --apo_pool.pending == 0)
            pthread_cond_signal(&apo_pool.done);
    }
    return NULL;
}

static void apo_pool_run(size_t n, apo_rows_fn fn, void *ctx, int threads) {
    if (threads <= 0) threads = apo_default_threads();
    if (threads > APO_MAX_THREADS) threads = APO_MAX_THREADS;
    if ((size_t)threads > n) threads = n ? (int)n : 1;
    if (threads <= 1) {
        if (n) fn(ctx, 0, n);
        return;
    }
    pthread_mutex_lock(&apo_pool_call_mu);
    pthread_mutex_lock(&apo_pool.mu);
    while (apo_pool.spawned < threads - 1) {
        int lane = apo_pool.spawned + 1;
        if (pthread_create(&apo_pool.tid[lane], NULL, apo_worker,
                           (void *)(intptr_t)lane) != 0)
            break;
        pthread_detach(apo_pool.tid[lane]);
        apo_pool.spawned++;
    }
    if (apo_pool.spawned < threads - 1) threads = apo_pool.spawned + 1;
    size_t base = n / (size_t)threads, rem = n % (size_t)threads, at = 0;
    for (int l = 0; l < threads; l++) {
        size_t len = base + ((size_t)l < rem ? 1 : 0);
        apo_pool.lo[l] = at;
        apo_pool.hi[l] = at + len;
        at += len;
    }
    apo_pool.fn = fn;
    apo_pool.ctx = ctx;
    apo_pool.nlane = threads;
    apo_pool.pending = threads - 1;
    apo_pool.gen++;
    pthread_cond_broadcast(&apo_pool.work);
    size_t lo0 = apo_pool.lo[0], hi0 = apo_pool.hi[0];
    pthread_mutex_unlock(&apo_pool.mu);
    if (hi0 > lo0) fn(ctx, lo0, hi0);
    pthread_mutex_lock(&apo_pool.mu);
    while (apo_pool.pending > 0)
        pthread_cond_wait(&apo_pool.done, &apo_pool.mu);
    pthread_mutex_unlock(&apo_pool.mu);
    pthread_mutex_unlock(&apo_pool_call_mu);
}

/* ======================================================================== */
/* FP8 128x128-block dequant                                                 */
/* ======================================================================== */

/* Rows [o0,o1) of c/fp8blk.h:115-131: out = bf16(e4m3(code) * scale of the
 * element's 128x128 block), one fp32 multiply then the RNE narrow. Partial
 * edge blocks use the edge scale. */
static void apo_dequant_rows(const uint8_t *w, const float *ws, uint16_t *out,
                             size_t K, size_t o0, size_t o1) {
    size_t nkb = apo_nblocks(K);
    for (size_t o = o0; o < o1; o++) {
        const float *srow = ws + (o / 128) * nkb;
        for (size_t k = 0; k < K; k++)
            out[o * K + k] = apo_bf16_bits(apo_e4m3_f32(w[o * K + k])
                                           * srow[k / 128]);
    }
}

void apo_fp8blk_dequant(const uint8_t *w, const float *ws, uint16_t *out,
                        size_t O, size_t K) {
    apo_dequant_rows(w, ws, out, K, 0, O);
}

typedef struct {
    const uint8_t *w;
    const float *ws;
    uint16_t *out;
    size_t K;
} ApoDeqJob;

/* Threaded leg: an exact 256-entry decode table replaces the per-code
 * decode (same values, apo_e4m3_f32 is exact), then one fp32 multiply and
 * the RNE narrow per element, exactly as the scalar rows. */
static float apo_e4m3_lut[256];
static pthread_once_t apo_lut_once = PTHREAD_ONCE_INIT;
static void apo_lut_init(void) {
    for (int c = 0; c < 256; c++) apo_e4m3_lut[c] = apo_e4m3_f32((uint8_t)c);
}

static void apo_dequant_rows_fast(void *vj, size_t o0, size_t o1) {
    const ApoDeqJob *j = (const ApoDeqJob *)vj;
    size_t K = j->K, nkb = apo_nblocks(K);
    for (size_t o = o0; o < o1; o++) {
        const uint8_t *wr = j->w + o * K;
        const float *srow = j->ws + (o / 128) * nkb;
        uint16_t *orow = j->out + o * K;
        for (size_t kb = 0; kb < nkb; kb++) {
            float s = srow[kb];
            size_t lo = kb * 128, hi = lo + 128 < K ? lo + 128 : K;
            for (size_t k = lo; k < hi; k++)
                orow[k] = apo_bf16_bits(apo_e4m3_lut[wr[k]] * s);
        }
    }
}

void apo_fp8blk_dequant_mt(const uint8_t *w, const float *ws, uint16_t *out,
                           size_t O, size_t K, int threads) {
    pthread_once(&apo_lut_once, apo_lut_init);
    ApoDeqJob j = { w, ws, out, K };
    apo_pool_run(O, apo_dequant_rows_fast, &j, threads);
}

/* ======================================================================== */
/* BF16 GEMV/GEMM                                                            */
/* ======================================================================== */

/* c/bf16.h:202-217: acc = +0.0f; for k ascending: acc += f32(W)*f32(x)
 * (product rounding, then add rounding; no FMA); y = bf16(acc). */
void apo_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                   size_t M, size_t O, size_t K) {
    for (size_t m = 0; m < M; m++)
        for (size_t o = 0; o < O; o++) {
            float acc = 0.0f;
            for (size_t k = 0; k < K; k++) {
                float p = apo_bf16_f32(w[o * K + k]) * apo_bf16_f32(x[m * K + k]);
                acc = acc + p;
            }
            y[m * O + o] = apo_bf16_bits(acc);
        }
}

void apo_bf16_gemm_absdot(const uint16_t *w, const uint16_t *x, double *a,
                          size_t M, size_t O, size_t K) {
    for (size_t m = 0; m < M; m++)
        for (size_t o = 0; o < O; o++) {
            double s = 0.0;
            for (size_t k = 0; k < K; k++)
                s += fabs((double)apo_bf16_f32(w[o * K + k])
                          * (double)apo_bf16_f32(x[m * K + k]));
            a[m * O + o] = s;
        }
}

typedef struct {
    const uint16_t *w;
    const float *xf;      /* widened x [M, K] */
    uint16_t *y;
    size_t M, O, K;
} ApoGemmJob;

#define APO_CHUNK 32

/* Scalar row body over pre-widened x (bitwise the anchor). */
static float apo_dot_seq(const uint16_t *wr, const float *xr, size_t k0,
                         size_t K, float acc) {
    for (size_t k = k0; k < K; k++) {
        float p = apo_bf16_f32(wr[k]) * xr[k];
        acc = acc + p;
    }
    return acc;
}

#if APO_X86
/* 8 exact bf16 -> fp32 widens (bits << 16). */
__attribute__((target("avx2")))
static inline __m256 apo_widen8(const uint16_t *p) {
    return _mm256_castsi256_ps(_mm256_slli_epi32(
        _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)p)), 16));
}

/* Products W[k..k+32) * x[k..k+32) staged with one fp32 rounding each
 * (vmulps == scalar mul), then added strictly in ascending k by the caller:
 * the staged-product pattern of c/bf16.h:444-500. */
__attribute__((target("avx2")))
static inline void apo_stage32(const uint16_t *wr, const float *xr, float *st) {
    for (int i = 0; i < APO_CHUNK; i += 8)
        _mm256_storeu_ps(st + i, _mm256_mul_ps(apo_widen8(wr + i),
                                               _mm256_loadu_ps(xr + i)));
}

/* GEMV rows, M == 1: eight independent row chains per pass (each chain is
 * the sequential sum for its row), c/bf16.h:506-572 structure. */
__attribute__((target("avx2")))
static void apo_gemv_rows_avx2(void *vj, size_t o0, size_t o1) {
    const ApoGemmJob *j = (const ApoGemmJob *)vj;
    const size_t K = j->K;
    const float *xf = j->xf;
    float st[8][APO_CHUNK];
    size_t o = o0;
    for (; o + 8 <= o1; o += 8) {
        float acc[8] = { 0, 0, 0, 0, 0, 0, 0, 0 };
        size_t k = 0;
        for (; k + APO_CHUNK <= K; k += APO_CHUNK) {
            for (int r = 0; r < 8; r++)
                apo_stage32(j->w + (o + r) * K + k, xf + k, st[r]);
            for (int i = 0; i < APO_CHUNK; i++) {
                acc[0] = acc[0] + st[0][i];
                acc[1] = acc[1] + st[1][i];
                acc[2] = acc[2] + st[2][i];
                acc[3] = acc[3] + st[3][i];
                acc[4] = acc[4] + st[4][i];
                acc[5] = acc[5] + st[5][i];
                acc[6] = acc[6] + st[6][i];
                acc[7] = acc[7] + st[7][i];
            }
        }
        for (int r = 0; r < 8; r++)
            j->y[o + r] = apo_bf16_bits(
                apo_dot_seq(j->w + (o + r) * K, xf, k, K, acc[r]));
    }
    for (; o < o1; o++) {
        float acc = 0.0f;
        size_t k = 0;
        for (; k + APO_CHUNK <= K; k += APO_CHUNK) {
            apo_stage32(j->w + o * K + k, xf + k, st[0]);
            for (int i = 0; i < APO_CHUNK; i++) acc = acc + st[0][i];
        }
        j->y[o] = apo_bf16_bits(apo_dot_seq(j->w + o * K, xf, k, K, acc));
    }
}

/* GEMM rows, M > 1: each widened W chunk is shared across up to four
 * activation rows (c/bf16.h:578-634 structure); per output the adds stay
 * strictly sequential in k, so y is M- and partition-independent. */
__attribute__((target("avx2")))
static void apo_gemm_rows_avx2(void *vj, size_t o0, size_t o1) {
    const ApoGemmJob *j = (const ApoGemmJob *)vj;
    const size_t K = j->K, M = j->M, O = j->O;
    float st[4][APO_CHUNK];
    for (size_t m0 = 0; m0 < M; m0 += 4) {
        size_t mc = M - m0 < 4 ? M - m0 : 4;
        for (size_t o = o0; o < o1; o++) {
            const uint16_t *wr = j->w + o * K;
            float acc[4] = { 0, 0, 0, 0 };
            size_t k = 0;
            for (; k + APO_CHUNK <= K; k += APO_CHUNK) {
                for (int i = 0; i < APO_CHUNK; i += 8) {
                    __m256 wv = apo_widen8(wr + k + i);
                    for (size_t r = 0; r < mc; r++)
                        _mm256_storeu_ps(st[r] + i, _mm256_mul_ps(wv,
                            _mm256_loadu_ps(j->xf + (m0 + r) * K + k + i)));
                }
                for (int i = 0; i < APO_CHUNK; i++)
                    for (size_t r = 0; r < mc; r++)
                        acc[r] = acc[r] + st[r][i];
            }
            for (size_t r = 0; r < mc; r++)
                j->y[(m0 + r) * O + o] = apo_bf16_bits(apo_dot_seq(
                    wr, j->xf + (m0 + r) * K, k, K, acc[r]));
        }
    }
}
#endif

static void apo_gemm_rows_scalar(void *vj, size_t o0, size_t o1) {
    const ApoGemmJob *j = (const ApoGemmJob *)vj;
    for (size_t m = 0; m < j->M; m++)
        for (size_t o = o0; o < o1; o++)
            j->y[m * j->O + o] = apo_bf16_bits(apo_dot_seq(
                j->w + o * j->K, j->xf + m * j->K, 0, j->K, 0.0f));
}

int apo_bf16_gemm_mt(const uint16_t *w, const uint16_t *x, uint16_t *y,
                     size_t M, size_t O, size_t K, int threads) {
    float *xf = (float *)malloc((M * K > 0 ? M * K : 1) * sizeof(float));
    if (!xf) return 1;
    for (size_t i = 0; i < M * K; i++) xf[i] = apo_bf16_f32(x[i]);
    ApoGemmJob j = { w, xf, y, M, O, K };
#if APO_X86
    if (__builtin_cpu_supports("avx2"))
        apo_pool_run(O, M == 1 ? apo_gemv_rows_avx2 : apo_gemm_rows_avx2, &j,
                     threads);
    else
#endif
        apo_pool_run(O, apo_gemm_rows_scalar, &j, threads);
    free(xf);
    return 0;
}

int apo_fp8blk_linear(const uint8_t *codes, const float *scales,
                      const uint16_t *x, uint16_t *y,
                      size_t M, size_t O, size_t K, int threads) {
    uint16_t *wb = (uint16_t *)malloc((O * K > 0 ? O * K : 1) * 2);
    if (!wb) return 1;
    int rc = 0;
    if (threads == 1) {
        apo_fp8blk_dequant(codes, scales, wb, O, K);
        apo_bf16_gemm(wb, x, y, M, O, K);
    } else {
        apo_fp8blk_dequant_mt(codes, scales, wb, O, K, threads);
        rc = apo_bf16_gemm_mt(wb, x, y, M, O, K, threads);
    }
    free(wb);
    return rc;
}

/* ======================================================================== */
/* SwiGLU expert, routing, combine                                           */
/* ======================================================================== */

/* c/gmhc.h:157-160 (numpy-stable form, libm expf). */
float apo_sigmoid_np(float x) {
    float e = expf(-fabsf(x));
    return x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
}

/* c/gmhc.h:165-185: numpy float32 pairwise sum. n < 8: sequential from
 * a[0]; n <= 128: eight strided accumulators, tree-combined, then the
 * sequential remainder; larger n: halves split at a multiple of 8. */
float apo_pw_sum(const float *a, size_t n) {
    if (n == 0) return 0.0f;
    if (n < 8) {
        float r = a[0];
        for (size_t i = 1; i < n; i++) r = r + a[i];
        return r;
    }
    if (n <= 128) {
        float r[8];
        for (int q = 0; q < 8; q++) r[q] = a[q];
        size_t i = 8;
        for (; i + 8 <= n; i += 8)
            for (int q = 0; q < 8; q++) r[q] = r[q] + a[i + q];
        float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; i++) s = s + a[i];
        return s;
    }
    size_t h = (n / 2) & ~(size_t)7;
    return apo_pw_sum(a, h) + apo_pw_sum(a + h, n - h);
}

/* c/gmoe.h:175-189 */
void apo_topk_stable(const float *row, int n, int k, int32_t *idx) {
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            int taken = 0;
            for (int q = 0; q < j; q++)
                if (idx[q] == i) { taken = 1; break; }
            if (taken) continue;
            if (best < 0 || row[i] > row[best]) best = i;
        }
        idx[j] = best;
    }
}

/* c/gmoe.h:168-173: fp32 dot of one gate row, strictly ascending k, from
 * +0, mul then add (the bf16 x bf16 products are exact in fp32). */
float apo_gate_dot(const uint16_t *wrow, const uint16_t *x, size_t k) {
    float acc = 0.0f;
    for (size_t i = 0; i < k; i++) {
        float p = apo_bf16_f32(wrow[i]) * apo_bf16_f32(x[i]);
        acc = acc + p;
    }
    return acc;
}

/* c/gmoe.h:191-208 (the reference router): logits by apo_gate_dot, scores
 * = numpy-stable sigmoid (c/gmhc.h:157-160), selection on scores + bias
 * only, stable top-k (ties -> lower id), w = the unbiased scores of the
 * selection, normalized by their numpy pairwise sum (c/gmhc.h:165-185)
 * + 1e-20 and scaled by route_scale. scores [E] out (may be NULL). */
void apo_gmoe_router(const uint16_t *gate_w, const float *gate_bias, int E,
                     size_t dim, int topk, float route_scale, const uint16_t *x,
                     float *scores, int32_t *idx, float *w) {
    float *sc = (float *)malloc((size_t)E * sizeof(float));
    float *b = (float *)malloc((size_t)E * sizeof(float));
    for (int e = 0; e < E; e++) {
        float logit = apo_gate_dot(gate_w + (size_t)e * dim, x, dim);
        sc[e] = apo_sigmoid_np(logit);
        b[e] = sc[e] + gate_bias[e];
    }
    apo_topk_stable(b, E, topk, idx);
    for (int j = 0; j < topk; j++) w[j] = sc[idx[j]];
    float sum = apo_pw_sum(w, (size_t)topk);
    for (int j = 0; j < topk; j++) w[j] = w[j] / (sum + 1e-20f) * route_scale;
    if (scores) memcpy(scores, sc, (size_t)E * sizeof(float));
    free(sc);
    free(b);
}

/* The router's selection and weights from given logits (the device router
 * computes logits as a GEMV; this is the part after them). */
void apo_gmoe_router_from_logits(const float *logits, const float *gate_bias, int E,
                                 int topk, float route_scale, float *scores,
                                 int32_t *idx, float *w) {
    float *sc = (float *)malloc((size_t)E * sizeof(float));
    float *b = (float *)malloc((size_t)E * sizeof(float));
    for (int e = 0; e < E; e++) {
        sc[e] = apo_sigmoid_np(logits[e]);
        b[e] = sc[e] + gate_bias[e];
    }
    apo_topk_stable(b, E, topk, idx);
    for (int j = 0; j < topk; j++) w[j] = sc[idx[j]];
    float sum = apo_pw_sum(w, (size_t)topk);
    for (int j = 0; j < topk; j++) w[j] = w[j] / (sum + 1e-20f) * route_scale;
    if (scores) memcpy(scores, sc, (size_t)E * sizeof(float));
    free(sc);
    free(b);
}

void apo_route_softmax(const float *logits, int E, int k, int32_t *idx,
                       float *w) {
    apo_topk_stable(logits, E, k, idx);
    float mx = logits[idx[0]];
    float s = 0.0f;
    for (int j = 0; j < k; j++) {
        w[j] = expf(logits[idx[j]] - mx);
        s = s + w[j];
    }
    for (int j = 0; j < k; j++) w[j] = w[j] / s;
}

/* c/gmoe.h:210-227: g = GEMV(wg,x), u = GEMV(wu,x) (bf16 outputs);
 * g = min(g, limit); u = clip(u, -limit, limit);
 * h = bf16(bf16(g * sigmoid(g)) * u); out = GEMV(wd, h). */
int apo_swiglu_expert(const uint16_t *wg, const uint16_t *wu,
                      const uint16_t *wd, const uint16_t *x,
                      size_t dim, size_t inter, float limit,
                      uint16_t *out, uint16_t *g_out, uint16_t *u_out,
                      uint16_t *h_out, int threads) {
    uint16_t *g = (uint16_t *)malloc(inter * 2);
    uint16_t *u = (uint16_t *)malloc(inter * 2);
    uint16_t *h = (uint16_t *)malloc(inter * 2);
    int rc = (!g || !u || !h);
    if (!rc) {
        if (threads == 1) {
            apo_bf16_gemm(wg, x, g, 1, inter, dim);
            apo_bf16_gemm(wu, x, u, 1, inter, dim);
        } else {
            rc |= apo_bf16_gemm_mt(wg, x, g, 1, inter, dim, threads);
            rc |= apo_bf16_gemm_mt(wu, x, u, 1, inter, dim, threads);
        }
        for (size_t i = 0; i < inter; i++) {
            float gv = apo_bf16_f32(g[i]), uv = apo_bf16_f32(u[i]);
            if (gv > limit) gv = limit;
            if (uv > limit) uv = limit;
            else if (uv < -limit) uv = -limit;
            float hv = apo_bf16_round(gv * apo_sigmoid_np(gv));
            h[i] = apo_bf16_bits(apo_bf16_round(hv * uv));
        }
        if (threads == 1) apo_bf16_gemm(wd, h, out, 1, dim, inter);
        else rc |= apo_bf16_gemm_mt(wd, h, out, 1, dim, inter, threads);
        if (g_out) memcpy(g_out, g, inter * 2);
        if (u_out) memcpy(u_out, u, inter * 2);
        if (h_out) memcpy(h_out, h, inter * 2);
    }
    free(g); free(u); free(h);
    return rc;
}

/* c/gcache.h:852-861 member order and sizes. */
ApoSlabLayout apo_slab_layout(size_t dim, size_t inter) {
    ApoSlabLayout L;
    size_t gw_b = inter * dim;
    size_t gs_b = apo_nblocks(inter) * apo_nblocks(dim) * sizeof(float);
    size_t dw_b = dim * inter;
    size_t ds_b = apo_nblocks(dim) * apo_nblocks(inter) * sizeof(float);
    L.gw = 0;
    L.gs = gw_b;
    L.uw = gw_b + gs_b;
    L.us = gw_b + gs_b + gw_b;
    L.dw = 2 * (gw_b + gs_b);
    L.ds = 2 * (gw_b + gs_b) + dw_b;
    L.bytes = 2 * (gw_b + gs_b) + dw_b + ds_b;
    return L;
}

/* c/gcache.h:413-426: three dequants into [gate | up | down]. */
void apo_slab_dequant(const uint8_t *slab, size_t dim, size_t inter,
                      uint16_t *payload, int threads) {
    ApoSlabLayout L = apo_slab_layout(dim, inter);
    const size_t n = inter * dim;
    if (threads == 1) {
        apo_fp8blk_dequant(slab + L.gw, (const float *)(slab + L.gs),
                           payload, inter, dim);
        apo_fp8blk_dequant(slab + L.uw, (const float *)(slab + L.us),
                           payload + n, inter, dim);
        apo_fp8blk_dequant(slab + L.dw, (const float *)(slab + L.ds),
                           payload + 2 * n, dim, inter);
    } else {
        apo_fp8blk_dequant_mt(slab + L.gw, (const float *)(slab + L.gs),
                              payload, inter, dim, threads);
        apo_fp8blk_dequant_mt(slab + L.uw, (const float *)(slab + L.us),
                              payload + n, inter, dim, threads);
        apo_fp8blk_dequant_mt(slab + L.dw, (const float *)(slab + L.ds),
                              payload + 2 * n, dim, inter, threads);
    }
}

/* c/gmoe.h:294-336 per token: the routed experts in ascending id (one bf16
 * rounding per add), then, when shared_slab is given, the shared expert's
 * output added last with one more rounding: out = bf16(y + sh) (no weight,
 * c/gmoe.h:325-336; the shared expert's intermediate is inter, as
 * n_shared_experts = 1 makes it, c/gmodel.h:963-964). */
static int apo_moe_loop(const uint8_t *const *slabs, int n_experts,
                        const uint8_t *shared_slab, size_t dim, size_t inter,
                        float limit, const uint16_t *x, size_t T, const int32_t *idx,
                        const float *w, int topk, uint16_t *out,
                        uint16_t *expert_out, uint16_t *shared_out, int threads) {
    const size_t pn = 3 * inter * dim;
    uint16_t **payload = (uint16_t **)calloc((size_t)n_experts, sizeof(*payload));
    float *y = (float *)malloc(dim * sizeof(float));
    uint16_t *eo = (uint16_t *)malloc(dim * 2);
    uint16_t *spl = shared_slab ? (uint16_t *)malloc(pn * 2) : NULL;
    int rc = (!payload || !y || !eo || (shared_slab && !spl));
    if (!rc && spl) apo_slab_dequant(shared_slab, dim, inter, spl, threads);
    for (size_t t = 0; t < T && !rc; t++) {
        const int32_t *it = idx + t * (size_t)topk;
        for (size_t i = 0; i < dim; i++) y[i] = 0.0f;
        /* c/gmoe.h:307-320: ascending expert id, first matching slot */
        for (int e = 0; e < n_experts && !rc; e++) {
            int slot = -1;
            for (int q = 0; q < topk; q++)
                if (it[q] == e) { slot = q; break; }
            if (slot < 0) continue;
            if (!payload[e]) {
                payload[e] = (uint16_t *)malloc(pn * 2);
                if (!payload[e]) { rc = 1; break; }
                apo_slab_dequant(slabs[e], dim, inter, payload[e], threads);
            }
            const uint16_t *pl = payload[e];
            rc |= apo_swiglu_expert(pl, pl + inter * dim, pl + 2 * inter * dim,
                                    x + t * dim, dim, inter, limit, eo,
                                    NULL, NULL, NULL, threads);
            if (expert_out)
                memcpy(expert_out + (t * (size_t)topk + (size_t)slot) * dim,
                       eo, dim * 2);
            float wt = w[t * (size_t)topk + (size_t)slot];
            for (size_t i = 0; i < dim; i++) {
                float contrib = apo_bf16_round(apo_bf16_f32(eo[i]) * wt);
                y[i] = apo_bf16_round(y[i] + contrib);
            }
        }
        if (spl && !rc) {
            rc |= apo_swiglu_expert(spl, spl + inter * dim, spl + 2 * inter * dim,
                                    x + t * dim, dim, inter, limit, eo,
                                    NULL, NULL, NULL, threads);
            if (shared_out) memcpy(shared_out + t * dim, eo, dim * 2);
            for (size_t i = 0; i < dim; i++) y[i] = y[i] + apo_bf16_f32(eo[i]);
        }
        for (size_t i = 0; i < dim; i++) out[t * dim + i] = apo_bf16_bits(y[i]);
    }
    if (payload)
        for (int e = 0; e < n_experts; e++) free(payload[e]);
    free(payload);
    free(y);
    free(eo);
    free(spl);
    return rc;
}

int apo_moe_forward(const uint8_t *const *slabs, int n_experts,
                    size_t dim, size_t inter, float limit,
                    const uint16_t *x, size_t T, const int32_t *idx,
                    const float *w, int topk, uint16_t *out,
                    uint16_t *expert_out, int threads) {
    return apo_moe_loop(slabs, n_experts, NULL, dim, inter, limit, x, T, idx, w, topk,
                        out, expert_out, NULL, threads);
}

int apo_moe_forward_shared(const uint8_t *const *slabs, int n_experts,
                           const uint8_t *shared_slab, size_t dim, size_t inter,
                           float limit, const uint16_t *x, size_t T, const int32_t *idx,
                           const float *w, int topk, uint16_t *out,
                           uint16_t *expert_out, uint16_t *shared_out, int threads) {
    return apo_moe_loop(slabs, n_experts, shared_slab, dim, inter, limit, x, T, idx, w,
                        topk, out, expert_out, shared_out, threads);
}

/* GEMM over many activation rows for the grouped checker: rows go in
 * blocks of 8, held transposed ([k][8] f32) so one vector holds the 8 rows'
 * k-th activations, and each output's 8 row sums advance together, lane r
 * being row r's strictly sequential k chain from +0 (one fp32 mul then
 * one add per k, as c/bf16.h:27-37): bitwise the scalar anchor, M times
 * faster than one chain at a time. Four weight rows share each block. */
typedef struct {
    const uint16_t *w;
    const float *xt;      /* [ceil(M/8)][K][8] widened, transposed x (zero pad) */
    uint16_t *y;
    size_t M, O, K;
} ApoRowvecJob;

static inline float apo_wf(const uint16_t *w, size_t i) { return apo_bf16_f32(w[i]); }

#if APO_X86
__attribute__((target("avx2")))
static void apo_gemm_rows_rowvec(void *vj, size_t o0, size_t o1) {
    const ApoRowvecJob *j = (const ApoRowvecJob *)vj;
    const size_t K = j->K, M = j->M, O = j->O;
    float res[4][8];
    /* the 4 weight rows of an o block widened once, interleaved [k][4] */
    float *wf = (float *)malloc(K * 4 * sizeof(float));
    if (!wf) abort();
    for (size_t o = o0; o < o1; o += 4) {
        const size_t oc = o1 - o < 4 ? o1 - o : 4;
        for (size_t q = 0; q < 4; q++) {
            const uint16_t *wr = j->w + (o + (q < oc ? q : 0)) * K;
            for (size_t k = 0; k < K; k++) wf[k * 4 + q] = apo_wf(wr, k);
        }
        for (size_t m0 = 0; m0 < M; m0 += 8) {
            const float *xb = j->xt + (m0 / 8) * K * 8;
            const size_t mc = M - m0 < 8 ? M - m0 : 8;
            __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
            for (size_t k = 0; k < K; k++) {
                const __m256 xv = _mm256_loadu_ps(xb + k * 8);
                const float *wk = wf + k * 4;
                a0 = _mm256_add_ps(a0, _mm256_mul_ps(_mm256_broadcast_ss(wk), xv));
                a1 = _mm256_add_ps(a1, _mm256_mul_ps(_mm256_broadcast_ss(wk + 1), xv));
                a2 = _mm256_add_ps(a2, _mm256_mul_ps(_mm256_broadcast_ss(wk + 2), xv));
                a3 = _mm256_add_ps(a3, _mm256_mul_ps(_mm256_broadcast_ss(wk + 3), xv));
            }
            _mm256_storeu_ps(res[0], a0);
            _mm256_storeu_ps(res[1], a1);
            _mm256_storeu_ps(res[2], a2);
            _mm256_storeu_ps(res[3], a3);
            for (size_t q = 0; q < oc; q++)
                for (size_t r = 0; r < mc; r++)
                    j->y[(m0 + r) * O + o + q] = apo_bf16_bits(res[q][r]);
        }
    }
    free(wf);
}
#endif

static void apo_gemm_rows_rowvec_scalar(void *vj, size_t o0, size_t o1) {
    const ApoRowvecJob *j = (const ApoRowvecJob *)vj;
    const size_t K = j->K;
    for (size_t m = 0; m < j->M; m++) {
        const float *xb = j->xt + (m / 8) * K * 8 + (m % 8);
        for (size_t o = o0; o < o1; o++) {
            float acc = 0.0f;
            for (size_t k = 0; k < K; k++) {
                float p = apo_wf(j->w + o * K, k) * xb[k * 8];
                acc = acc + p;
            }
            j->y[m * j->O + o] = apo_bf16_bits(acc);
        }
    }
}

static int apo_gemm_rowvec(const uint16_t *w, const uint16_t *x, uint16_t *y,
                           size_t M, size_t O, size_t K, int threads) {
    const size_t nb = (M + 7) / 8;
    float *xt = (float *)calloc(nb * K * 8 > 0 ? nb * K * 8 : 1, sizeof(float));
    if (!xt) return 1;
    for (size_t m = 0; m < M; m++)
        for (size_t k = 0; k < K; k++)
            xt[(m / 8) * K * 8 + k * 8 + (m % 8)] = apo_bf16_f32(x[m * K + k]);
    ApoRowvecJob j = { w, xt, y, M, O, K };
#if APO_X86
    if (__builtin_cpu_supports("avx2"))
        apo_pool_run(O, apo_gemm_rows_rowvec, &j, threads);
    else
#endif
        apo_pool_run(O, apo_gemm_rows_rowvec_scalar, &j, threads);
    free(xt);
    return 0;
}

/* The same GEMM with every dot product summed in f64 (the bf16 x bf16
 * products are exact; an f64 sum of K <= 16384 of them is within ~2^-39
 * relative of the exact sum), then rounded to f32 and to bf16: a yardstick
 * free of any fp32 summation order, not a reference function. Rows in
 * blocks of 4 (one f64 vector), 4 weight rows per block. */
typedef struct {
    const uint16_t *w;
    const double *xt;     /* [ceil(M/4)][K][4] */
    uint16_t *y;
    size_t M, O, K;
} ApoRowvec64Job;

#if APO_X86
__attribute__((target("avx2")))
static void apo_gemm_rows_rowvec64(void *vj, size_t o0, size_t o1) {
    const ApoRowvec64Job *j = (const ApoRowvec64Job *)vj;
    const size_t K = j->K, M = j->M, O = j->O;
    double res[4][4];
    double *wf = (double *)malloc(K * 4 * sizeof(double));
    if (!wf) abort();
    for (size_t o = o0; o < o1; o += 4) {
        const size_t oc = o1 - o < 4 ? o1 - o : 4;
        for (size_t q = 0; q < 4; q++) {
            const uint16_t *wr = j->w + (o + (q < oc ? q : 0)) * K;
            for (size_t k = 0; k < K; k++) wf[k * 4 + q] = (double)apo_wf(wr, k);
        }
        for (size_t m0 = 0; m0 < M; m0 += 4) {
            const double *xb = j->xt + (m0 / 4) * K * 4;
            const size_t mc = M - m0 < 4 ? M - m0 : 4;
            __m256d a0 = _mm256_setzero_pd(), a1 = a0, a2 = a0, a3 = a0;
            for (size_t k = 0; k < K; k++) {
                const __m256d xv = _mm256_loadu_pd(xb + k * 4);
                const double *wk = wf + k * 4;
                a0 = _mm256_add_pd(a0, _mm256_mul_pd(_mm256_broadcast_sd(wk), xv));
                a1 = _mm256_add_pd(a1, _mm256_mul_pd(_mm256_broadcast_sd(wk + 1), xv));
                a2 = _mm256_add_pd(a2, _mm256_mul_pd(_mm256_broadcast_sd(wk + 2), xv));
                a3 = _mm256_add_pd(a3, _mm256_mul_pd(_mm256_broadcast_sd(wk + 3), xv));
            }
            _mm256_storeu_pd(res[0], a0);
            _mm256_storeu_pd(res[1], a1);
            _mm256_storeu_pd(res[2], a2);
            _mm256_storeu_pd(res[3], a3);
            for (size_t q = 0; q < oc; q++)
                for (size_t r = 0; r < mc; r++)
                    j->y[(m0 + r) * O + o + q] = apo_bf16_bits((float)res[q][r]);
        }
    }
    free(wf);
}
#endif

static void apo_gemm_rows_rowvec64_scalar(void *vj, size_t o0, size_t o1) {
    const ApoRowvec64Job *j = (const ApoRowvec64Job *)vj;
    const size_t K = j->K;
    for (size_t m = 0; m < j->M; m++) {
        const double *xb = j->xt + (m / 4) * K * 4 + (m % 4);
        for (size_t o = o0; o < o1; o++) {
            double acc = 0.0;
            for (size_t k = 0; k < K; k++) acc += (double)apo_wf(j->w + o * K, k) * xb[k * 4];
            j->y[m * j->O + o] = apo_bf16_bits((float)acc);
        }
    }
}

static int apo_gemm_rowvec64(const uint16_t *w, const uint16_t *x, uint16_t *y,
                             size_t M, size_t O, size_t K, int threads) {
    const size_t nb = (M + 3) / 4;
    double *xt = (double *)calloc(nb * K * 4 > 0 ? nb * K * 4 : 1, sizeof(double));
    if (!xt) return 1;
    for (size_t m = 0; m < M; m++)
        for (size_t k = 0; k < K; k++)
            xt[(m / 4) * K * 4 + k * 4 + (m % 4)] = (double)apo_bf16_f32(x[m * K + k]);
    ApoRowvec64Job j = { w, xt, y, M, O, K };
#if APO_X86
    if (__builtin_cpu_supports("avx2"))
        apo_pool_run(O, apo_gemm_rows_rowvec64, &j, threads);
    else
#endif
        apo_pool_run(O, apo_gemm_rows_rowvec64_scalar, &j, threads);
    free(xt);
    return 0;
}

/* apo_moe_forward computed expert by expert, for checks at full size: each
 * used expert is dequantized once and its tokens run as one M-row GEMM per
 * matrix (c/bf16.h:27-37 makes every output row M-independent, so the
 * per-pair outputs are the per-token loop's bits), the per-pair outputs
 * are kept, and each token's ascending-expert combine (c/gmoe.h:307-320)
 * follows. Bitwise equal to apo_moe_forward. */
static int apo_moe_grouped(const uint8_t *const *slabs, int n_experts,
                           const uint8_t *shared_slab, size_t dim, size_t inter,
                           float limit,
                           const uint16_t *x, size_t T, const int32_t *idx,
                           const float *w, int topk, uint16_t *out,
                           uint16_t *expert_out, double *floor_out, int threads,
                           int sums64) {
    int (*gemm)(const uint16_t *, const uint16_t *, uint16_t *, size_t, size_t, size_t,
                int) = sums64 ? apo_gemm_rowvec64 : apo_gemm_rowvec;
    const size_t P = T * (size_t)topk, pn = 3 * inter * dim;
    int rc = 0;
    /* kept pairs: the first slot of each expert id in a token */
    int32_t *keep = (int32_t *)malloc((P ? P : 1) * sizeof(int32_t));
    size_t *cnt = (size_t *)calloc((size_t)n_experts + 1, sizeof(size_t));
    size_t *list = (size_t *)malloc((P ? P : 1) * sizeof(size_t));
    uint16_t *eo = expert_out ? expert_out
                              : (uint16_t *)malloc((P ? P : 1) * dim * 2);
    uint16_t *payload = (uint16_t *)malloc(pn * 2);
    /* floor_out: |down weights| of the current expert, and per pair the
     * expert-output floor F[j] = sum_i |h_i * wd[j,i]| (bf16) */
    uint16_t *dabs = floor_out ? (uint16_t *)malloc(dim * inter * 2) : NULL;
    uint16_t *fe = floor_out ? (uint16_t *)malloc((P ? P : 1) * dim * 2) : NULL;
    if (!keep || !cnt || !list || !eo || !payload || (floor_out && (!dabs || !fe))) rc = 1;
    for (size_t p = 0; p < P && !rc; p++) {
        const size_t t = p / (size_t)topk, j = p % (size_t)topk;
        const int32_t e = idx[p];
        int ok = e >= 0 && e < n_experts;
        for (size_t jj = 0; jj < j && ok; jj++)
            if (idx[t * (size_t)topk + jj] == e) ok = 0;
        keep[p] = ok ? e : -1;
        if (ok) cnt[e + 1]++;
    }
    for (int e = 0; e < n_experts && !rc; e++) cnt[e + 1] += cnt[e];
    if (!rc) {
        size_t *at = (size_t *)malloc(((size_t)n_experts + 1) * sizeof(size_t));
        if (!at) rc = 1;
        else {
            memcpy(at, cnt, ((size_t)n_experts + 1) * sizeof(size_t));
            for (size_t p = 0; p < P; p++)
                if (keep[p] >= 0) list[at[keep[p]]++] = p;
            free(at);
        }
    }
    for (int e = 0; e < n_experts && !rc; e++) {
        const size_t M = cnt[e + 1] - cnt[e];
        if (!M) continue;
        const size_t *pl = list + cnt[e];
        uint16_t *xe = (uint16_t *)malloc(M * dim * 2);
        uint16_t *g = (uint16_t *)malloc(M * inter * 2);
        uint16_t *u = (uint16_t *)malloc(M * inter * 2);
        uint16_t *oe = (uint16_t *)malloc(M * dim * 2);
        if (!xe || !g || !u || !oe) rc = 1;
        if (!rc) {
            apo_slab_dequant(slabs[e], dim, inter, payload, threads);
            for (size_t m = 0; m < M; m++)
                memcpy(xe + m * dim, x + (pl[m] / (size_t)topk) * dim, dim * 2);
            rc |= gemm(payload, xe, g, M, inter, dim, threads);
            rc |= gemm(payload + inter * dim, xe, u, M, inter, dim, threads);
            /* c/gmoe.h:217-225, the same steps as apo_swiglu_expert */
            for (size_t i = 0; i < M * inter; i++) {
                float gv = apo_bf16_f32(g[i]), uv = apo_bf16_f32(u[i]);
                if (gv > limit) gv = limit;
                if (uv > limit) uv = limit;
                else if (uv < -limit) uv = -limit;
                float hv = apo_bf16_round(gv * apo_sigmoid_np(gv));
                g[i] = apo_bf16_bits(apo_bf16_round(hv * uv));
            }
            rc |= gemm(payload + 2 * inter * dim, g, oe, M, dim, inter, threads);
            for (size_t m = 0; m < M; m++)
                memcpy(eo + pl[m] * dim, oe + m * dim, dim * 2);
            if (floor_out && !rc) {
                /* |h| . |wd|^T: the sum of the down GEMM's term magnitudes */
                const uint16_t *pd = payload + 2 * inter * dim;
                for (size_t i = 0; i < dim * inter; i++) dabs[i] = pd[i] & 0x7fffu;
                for (size_t i = 0; i < M * inter; i++) g[i] &= 0x7fffu;
                rc |= apo_gemm_rowvec64(dabs, g, oe, M, dim, inter, threads);
                for (size_t m = 0; m < M; m++)
                    memcpy(fe + pl[m] * dim, oe + m * dim, dim * 2);
            }
        }
        free(xe); free(g); free(u); free(oe);
    }
    /* the shared expert over all T tokens (c/gmoe.h:325-336): its output
     * sh [T, dim] and, for floor_out, its expert-output floor */
    uint16_t *sh = shared_slab ? (uint16_t *)malloc((T ? T : 1) * dim * 2) : NULL;
    uint16_t *fsh = shared_slab && floor_out ? (uint16_t *)malloc((T ? T : 1) * dim * 2)
                                             : NULL;
    if (shared_slab && (!sh || (floor_out && !fsh))) rc = 1;
    if (shared_slab && !rc && T) {
        uint16_t *g = (uint16_t *)malloc(T * inter * 2);
        uint16_t *u = (uint16_t *)malloc(T * inter * 2);
        if (!g || !u) rc = 1;
        if (!rc) {
            apo_slab_dequant(shared_slab, dim, inter, payload, threads);
            rc |= gemm(payload, x, g, T, inter, dim, threads);
            rc |= gemm(payload + inter * dim, x, u, T, inter, dim, threads);
            for (size_t i = 0; i < T * inter; i++) {
                float gv = apo_bf16_f32(g[i]), uv = apo_bf16_f32(u[i]);
                if (gv > limit) gv = limit;
                if (uv > limit) uv = limit;
                else if (uv < -limit) uv = -limit;
                float hv = apo_bf16_round(gv * apo_sigmoid_np(gv));
                g[i] = apo_bf16_bits(apo_bf16_round(hv * uv));
            }
            rc |= gemm(payload + 2 * inter * dim, g, sh, T, dim, inter, threads);
            if (floor_out && !rc) {
                const uint16_t *pd = payload + 2 * inter * dim;
                for (size_t i = 0; i < dim * inter; i++) dabs[i] = pd[i] & 0x7fffu;
                for (size_t i = 0; i < T * inter; i++) g[i] &= 0x7fffu;
                rc |= apo_gemm_rowvec64(dabs, g, fsh, T, dim, inter, threads);
            }
        }
        free(g); free(u);
    }
    /* c/gmoe.h:307-320 per token: ascending expert id over its kept pairs */
    float *y = (float *)malloc(dim * sizeof(float));
    if (!y) rc = 1;
    for (size_t t = 0; t < T && !rc; t++) {
        for (size_t i = 0; i < dim; i++) y[i] = 0.0f;
        int last = -1;
        for (;;) {
            size_t best = P;
            for (int j = 0; j < topk; j++) {
                const size_t p = t * (size_t)topk + (size_t)j;
                if (keep[p] > last && (best == P || keep[p] < keep[best])) best = p;
            }
            if (best == P) break;
            last = keep[best];
            const uint16_t *o = eo + best * dim;
            const float wt = w[best];
            for (size_t i = 0; i < dim; i++) {
                float contrib = apo_bf16_round(apo_bf16_f32(o[i]) * wt);
                y[i] = apo_bf16_round(y[i] + contrib);
            }
            if (floor_out)
                for (size_t i = 0; i < dim; i++)
                    floor_out[t * dim + i] += fabs((double)wt)
                                              * (double)apo_bf16_f32(fe[best * dim + i]);
        }
        if (sh) {
            for (size_t i = 0; i < dim; i++) y[i] = y[i] + apo_bf16_f32(sh[t * dim + i]);
            if (floor_out)
                for (size_t i = 0; i < dim; i++)
                    floor_out[t * dim + i] += (double)apo_bf16_f32(fsh[t * dim + i]);
        }
        for (size_t i = 0; i < dim; i++) out[t * dim + i] = apo_bf16_bits(y[i]);
    }
    free(y);
    free(sh); free(fsh);
    free(dabs); free(fe);
    free(keep); free(cnt); free(list); free(payload);
    if (!expert_out) free(eo);
    return rc;
}

int apo_moe_forward_grouped(const uint8_t *const *slabs, int n_experts,
                            const uint8_t *shared_slab, size_t dim, size_t inter,
                            float limit, const uint16_t *x, size_t T, const int32_t *idx,
                            const float *w, int topk, uint16_t *out,
                            uint16_t *expert_out, int threads) {
    return apo_moe_grouped(slabs, n_experts, shared_slab, dim, inter, limit, x, T, idx, w,
                           topk, out, expert_out, NULL, threads, 0);
}

int apo_moe_floor_grouped(const uint8_t *const *slabs, int n_experts,
                          const uint8_t *shared_slab, size_t dim, size_t inter,
                          float limit, const uint16_t *x, size_t T, const int32_t *idx,
                          const float *w, int topk, uint16_t *out,
                          double *floor_out, int threads) {
    for (size_t i = 0; i < T * dim; i++) floor_out[i] = 0.0;
    return apo_moe_grouped(slabs, n_experts, shared_slab, dim, inter, limit, x, T, idx, w,
                           topk, out, NULL, floor_out, threads, 0);
}

int apo_moe_chain64_grouped(const uint8_t *const *slabs, int n_experts,
                            const uint8_t *shared_slab, size_t dim, size_t inter,
                            float limit, const uint16_t *x, size_t T, const int32_t *idx,
                            const float *w, int topk, uint16_t *out,
                            uint16_t *expert_out, int threads) {
    return apo_moe_grouped(slabs, n_experts, shared_slab, dim, inter, limit, x, T, idx, w,
                           topk, out, expert_out, NULL, threads, 1);
}
