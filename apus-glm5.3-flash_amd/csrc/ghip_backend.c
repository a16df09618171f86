/*
 * ghip_backend.c — the C host layer of the MI355X backend (C11 over the HIP
 * runtime C API). Implements include/backend_hip.h: the hook table and its
 * enable/disable lifecycle, region registration (device mirrors of
 * model-owned weights), counters, the direct and device-pointer entry
 * points, the HBM expert slab store and the MoE decode entry points.
 *
 * Kernels live in the .hip units and are reached only through the launchers
 * of ghip_internal.h. Nothing here computes on the CPU: when the device or a
 * launch is unavailable an entry point returns nonzero and records why
 * (apus_ghip_last_error); the hook contract then lets the engine run its own
 * CPU kernel (c/bf16.h:717-719, c/gdsa.h:529-531).
 *
 * Reference counterparts: c/backend_gmetal.mm:378-487 (init, floors, hook
 * trampolines, region wraps), c/gcache.h:832-1004 (store layout/open).
 */
#include "backend_hip.h"
#include "apus_synth.h"
#include "ghip_internal.h"

#include <hip/hip_runtime_api.h>
#include <fcntl.h>
#include <pthread.h>
#include <semaphore.h>
#include <stdarg.h>
#include <unistd.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* weak default of the hook table (an engine TU may define the strong one) */
__attribute__((weak)) ApusGhipHooks apus_ghip_hooks;

#define GHIP_MAX_TOPK 16
#define GHIP_HW_SLOTS (GHIP_MAX_TOPK + 1)   /* routed slots + the shared expert */

/* ------------------------------------------------------------------------ */
/* state                                                                    */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint8_t *host;
    size_t len;
    void *dev;
} GhipRegion;

typedef struct {
    const void *dev;
    size_t n;
    int slot;                    /* index into the flag pool */
} GhipScan;

#define GHIP_SCAN_SLOTS 4096

static struct {
    int inited, enabled, device;
    uint32_t n_cu;               /* CU count rounded up to the 8 XCDs */
    uint32_t n_cu_dev;           /* the device's CU count */
    hipStream_t stream;
    /* grow-only staging (device) */
    void *d_w, *d_s, *d_x, *d_y;
    size_t cap_w, cap_s, cap_x, cap_y;
    uint32_t *d_flag;            /* ephemeral NaN-scan flag */
    uint32_t *d_flags;           /* pool of cached scan flags */
    int n_scan;
    GhipScan scan[GHIP_SCAN_SLOTS];
    GhipRegion *reg;
    size_t nreg, capreg;
    /* env floors (read once at enable) */
    size_t min_kb, fp8_min_kb;
    long max_m;
    /* counters */
    uint64_t bytes_wrapped, bytes_pinned, dispatches, off_bf16, off_fp8;
    uint64_t h2d, d2h;
    /* caller-owned timing events (apus_ghip_set_trace_events), n = 0: off */
    hipEvent_t trace_ev[8];
    int trace_n;
    /* K4 prefill workspace (process-wide, grow-only) and host staging */
    GhipMoePrefillWs pf;
    size_t pf_cap[8];
    void *pf_x, *pf_idx, *pf_w, *pf_out;
    size_t pf_cap_x, pf_cap_idx, pf_cap_w, pf_cap_out;
    int pf_inited;
} G;

static _Thread_local char g_err[512];

static void ghip_seterr(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

const char *apus_ghip_last_error(void) { return g_err; }

#define HIPCHK(call)                                                       \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) {                                            \
            ghip_seterr("%s: %s (%s:%d)", #call, hipGetErrorString(e_),    \
                        __FILE__, __LINE__);                               \
            return 1;                                                      \
        }                                                                  \
    } while (0)

static long env_long(const char *name, long dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    return strtol(v, NULL, 10);
}

/* Device selection and backend stream (default priority). */
static int ghip_init(void) {
    if (G.inited) return 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        ghip_seterr("no HIP device (%s)",
                    e != hipSuccess ? hipGetErrorString(e) : "count 0");
        return 1;
    }
    int dev = (int)env_long("APUS_GHIP_DEVICE", 0);
    if (dev < 0 || dev >= n) {
        ghip_seterr("APUS_GHIP_DEVICE=%d out of range (%d devices)", dev, n);
        return 1;
    }
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, dev));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        ghip_seterr("device %d is %s; this backend is built for gfx950", dev,
                    prop.gcnArchName);
        return 1;
    }
    HIPCHK(hipSetDevice(dev));
    HIPCHK(hipStreamCreate(&G.stream));
    int ncu = 0;
    HIPCHK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    if (ncu <= 0) {
        ghip_seterr("device %d reports no compute units", dev);
        return 1;
    }
    G.n_cu = (uint32_t)((ncu + 7) / 8 * 8);
    G.n_cu_dev = (uint32_t)ncu;
    HIPCHK(ghip_moe_decode_init());
    HIPCHK(ghip_linear_init(G.n_cu));
    HIPCHK(ghip_moe_prefill_init());
    G.pf.n_cu = G.n_cu;
    G.pf_inited = 1;
    /* the allocation-free prefill's scratch: its device address, taken once
     * here with the device current */
    HIPCHK(ghip_pf_scratch_init(dev));
    HIPCHK(hipMalloc((void **)&G.d_flag, 256));
    {
        /* word 0: the per-call NaN-scan flag; word 1: a constant 1 (the
         * exact-decode flag of exact = 1), written synchronously here */
        const uint32_t w01[2] = {0u, 1u};
        HIPCHK(hipMemcpy(G.d_flag, w01, sizeof w01, hipMemcpyHostToDevice));
    }
    HIPCHK(hipMalloc((void **)&G.d_flags, GHIP_SCAN_SLOTS * sizeof(uint32_t)));
    HIPCHK(hipMemset(G.d_flags, 0, GHIP_SCAN_SLOTS * sizeof(uint32_t)));
    G.device = dev;
    G.inited = 1;
    return 0;
}

static int grow(void **p, size_t *cap, size_t need) {
    if (need <= *cap) return 0;
    size_t nc = need < 4096 ? 4096 : need;
    nc = (nc + 4095) & ~(size_t)4095;
    if (*p) {
        HIPCHK(hipStreamSynchronize(G.stream));
        HIPCHK(hipFree(*p));
        *p = NULL;
        *cap = 0;
    }
    HIPCHK(hipMalloc(p, nc));
    *cap = nc;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* regions                                                                  */
/* ------------------------------------------------------------------------ */

/* Device address of host range [p, p+n) when a registered region covers it
 * (sub-ranges included, as c/backend_gmetal.mm:240-251). */
static void *region_find(const void *p, size_t n) {
    const uint8_t *q = (const uint8_t *)p;
    for (size_t i = 0; i < G.nreg; i++) {
        const GhipRegion *r = &G.reg[i];
        if (q >= r->host && q + n <= r->host + r->len && n <= r->len)
            return (uint8_t *)r->dev + (q - r->host);
    }
    return NULL;
}

int apus_ghip_register_region(const void *ptr, size_t len) {
    if (!G.enabled || !ptr || len == 0) {
        ghip_seterr("register_region: backend disabled or empty range");
        return 1;
    }
    for (size_t i = 0; i < G.nreg; i++)
        if (G.reg[i].host == ptr) return 0;          /* idempotent */
    if (G.nreg == G.capreg) {
        size_t nc = G.capreg ? 2 * G.capreg : 64;
        GhipRegion *nr = (GhipRegion *)realloc(G.reg, nc * sizeof *nr);
        if (!nr) { ghip_seterr("register_region: out of host memory"); return 1; }
        G.reg = nr;
        G.capreg = nc;
    }
    void *d = NULL;
    HIPCHK(hipMalloc(&d, len));
    hipError_t e = hipMemcpy(d, ptr, len, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(d);
        ghip_seterr("register_region: H2D %s", hipGetErrorString(e));
        return 1;
    }
    G.reg[G.nreg].host = (const uint8_t *)ptr;
    G.reg[G.nreg].len = len;
    G.reg[G.nreg].dev = d;
    G.nreg++;
    G.bytes_pinned += len;
    G.h2d += len;
    return 0;
}

void apus_ghip_unregister_region(const void *ptr) {
    for (size_t i = 0; i < G.nreg; i++) {
        if (G.reg[i].host != ptr) continue;
        GhipRegion r = G.reg[i];
        hipStreamSynchronize(G.stream);
        /* drop cached scans that point into this region */
        for (int s = 0; s < G.n_scan; s++) {
            const uint8_t *d = (const uint8_t *)G.scan[s].dev;
            if (d >= (uint8_t *)r.dev && d < (uint8_t *)r.dev + r.len)
                G.scan[s].dev = NULL;
        }
        hipFree(r.dev);
        G.bytes_pinned -= r.len;
        G.reg[i] = G.reg[--G.nreg];
        return;
    }
}

/* Cached NaN-code scan of resident device codes: returns a device flag
 * (u32, nonzero = exact decode needed), or NULL when the pool is full. */
static const uint32_t *scan_cached(const void *dcodes, size_t n) {
    for (int s = 0; s < G.n_scan; s++)
        if (G.scan[s].dev == dcodes && G.scan[s].n == n)
            return G.d_flags + G.scan[s].slot;
    if (G.n_scan >= GHIP_SCAN_SLOTS) return NULL;
    int slot = G.n_scan;
    if (ghip_launch_fill_u32(G.d_flags + slot, 1, 0u, G.stream) != hipSuccess
        || ghip_launch_nan_scan((const uint8_t *)dcodes, n, G.d_flags + slot,
                                G.stream) != hipSuccess)
        return NULL;
    G.scan[slot].dev = dcodes;
    G.scan[slot].n = n;
    G.scan[slot].slot = slot;
    G.n_scan++;
    return G.d_flags + slot;
}

/* ------------------------------------------------------------------------ */
/* lifecycle                                                                */
/* ------------------------------------------------------------------------ */

static int hook_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                          size_t M, size_t O, size_t K);
static int hook_fp8blk_linear(const uint8_t *codes, const float *scales,
                              const uint16_t *x, uint16_t *y, size_t M,
                              size_t O, size_t K);

int apus_ghip_enable(char *err, size_t errcap) {
    if (G.enabled) return 0;
    if (ghip_init()) {
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return 1;
    }
    long v = env_long("APUS_GHIP_MIN_KB", 0);
    G.min_kb = v > 0 ? (size_t)v : 0;
    v = env_long("APUS_GHIP_FP8_MIN_KB", 0);
    G.fp8_min_kb = v > 0 ? (size_t)v : 0;
    G.max_m = env_long("APUS_GHIP_MAX_M", 0);
    apus_ghip_hooks.bf16_gemm = hook_bf16_gemm;
    apus_ghip_hooks.fp8blk_linear = hook_fp8blk_linear;
    G.enabled = 1;
    return 0;
}

void apus_ghip_disable(void) {
    apus_ghip_hooks.bf16_gemm = NULL;
    apus_ghip_hooks.fp8blk_linear = NULL;
    if (!G.enabled) return;
    hipStreamSynchronize(G.stream);
    while (G.nreg) apus_ghip_unregister_region(G.reg[G.nreg - 1].host);
    free(G.reg);
    G.reg = NULL;
    G.capreg = 0;
    G.n_scan = 0;
    hipMemset(G.d_flags, 0, GHIP_SCAN_SLOTS * sizeof(uint32_t));
    void **bufs[4] = { &G.d_w, &G.d_s, &G.d_x, &G.d_y };
    size_t *caps[4] = { &G.cap_w, &G.cap_s, &G.cap_x, &G.cap_y };
    for (int i = 0; i < 4; i++) {
        if (*bufs[i]) hipFree(*bufs[i]);
        *bufs[i] = NULL;
        *caps[i] = 0;
    }
    G.enabled = 0;
}

int apus_ghip_is_enabled(void) { return G.enabled; }

uint64_t apus_ghip_bytes_wrapped(void) { return G.bytes_wrapped; }
uint64_t apus_ghip_bytes_pinned(void) { return G.bytes_pinned; }
uint64_t apus_ghip_dispatches(void) { return G.dispatches; }
uint64_t apus_ghip_offload_bf16(void) { return G.off_bf16; }
uint64_t apus_ghip_offload_fp8blk(void) { return G.off_fp8; }
uint64_t apus_ghip_bytes_h2d(void) { return G.h2d; }
uint64_t apus_ghip_bytes_d2h(void) { return G.d2h; }

/* ------------------------------------------------------------------------ */
/* host-pointer entry points                                                */
/* ------------------------------------------------------------------------ */

static int h2d(void *d, const void *h, size_t n) {
    if (n == 0) return 0;
    HIPCHK(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, G.stream));
    G.h2d += n;
    return 0;
}

/* Device address for a weight range: the registered mirror, else an upload
 * into the given staging buffer. */
static const void *weight_dev(const void *h, size_t n, void **stage,
                              size_t *cap) {
    void *d = region_find(h, n);
    if (d) return d;
    if (grow(stage, cap, n) || h2d(*stage, h, n)) return NULL;
    G.bytes_wrapped += n;
    return *stage;
}

static int sync_out(void *h, const void *d, size_t n) {
    HIPCHK(hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, G.stream));
    HIPCHK(hipStreamSynchronize(G.stream));
    G.d2h += n;
    return 0;
}

static int check_sizes(size_t M, size_t O, size_t K) {
    if (M == 0 || O == 0 || K == 0) {
        ghip_seterr("empty shape M=%zu O=%zu K=%zu", M, O, K);
        return 1;
    }
    if (O > 0x7fffffffu || K > 0x7fffffffu || M > 0x7fffffffu) {
        ghip_seterr("shape too large M=%zu O=%zu K=%zu", M, O, K);
        return 1;
    }
    return 0;
}

int apus_ghip_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                        size_t M, size_t O, size_t K) {
    if (ghip_init() || check_sizes(M, O, K)) return 1;
    const void *dw = weight_dev(w, O * K * 2, &G.d_w, &G.cap_w);
    if (!dw) return 1;
    if (grow(&G.d_x, &G.cap_x, M * K * 2) || grow(&G.d_y, &G.cap_y, M * O * 2)
        || h2d(G.d_x, x, M * K * 2))
        return 1;
    HIPCHK(ghip_launch_bf16_linear((const uint16_t *)dw, (const uint16_t *)G.d_x,
                                   (uint16_t *)G.d_y, M, O, K, NULL, G.stream));
    G.dispatches++;
    if (sync_out(y, G.d_y, M * O * 2)) return 1;
    G.off_bf16++;
    return 0;
}

int apus_ghip_fp8blk_linear(const uint8_t *codes, const float *scales,
                            const uint16_t *x, uint16_t *y,
                            size_t M, size_t O, size_t K) {
    if (ghip_init() || check_sizes(M, O, K)) return 1;
    size_t nsb = ((O + 127) / 128) * ((K + 127) / 128) * sizeof(float);
    int reg = region_find(codes, O * K) != NULL;
    const void *dc = weight_dev(codes, O * K, &G.d_w, &G.cap_w);
    const void *ds = dc ? weight_dev(scales, nsb, &G.d_s, &G.cap_s) : NULL;
    if (!dc || !ds) return 1;
    const uint32_t *flag = reg ? scan_cached(dc, O * K) : NULL;
    if (!flag) {
        HIPCHK(ghip_launch_fill_u32(G.d_flag, 1, 0u, G.stream));
        HIPCHK(ghip_launch_nan_scan((const uint8_t *)dc, O * K, G.d_flag,
                                    G.stream));
        flag = G.d_flag;
    }
    if (grow(&G.d_x, &G.cap_x, M * K * 2) || grow(&G.d_y, &G.cap_y, M * O * 2)
        || h2d(G.d_x, x, M * K * 2))
        return 1;
    HIPCHK(ghip_launch_fp8_linear((const uint8_t *)dc, (const float *)ds,
                                  (const uint16_t *)G.d_x, (uint16_t *)G.d_y,
                                  M, O, K, flag, NULL, G.stream));
    G.dispatches++;
    if (sync_out(y, G.d_y, M * O * 2)) return 1;
    G.off_fp8++;
    return 0;
}

int apus_ghip_fp8blk_dequant(const uint8_t *codes, const float *scales,
                             uint16_t *out, size_t O, size_t K) {
    if (ghip_init() || check_sizes(1, O, K)) return 1;
    size_t nsb = ((O + 127) / 128) * ((K + 127) / 128) * sizeof(float);
    const void *dc = weight_dev(codes, O * K, &G.d_w, &G.cap_w);
    const void *ds = dc ? weight_dev(scales, nsb, &G.d_s, &G.cap_s) : NULL;
    if (!dc || !ds || grow(&G.d_y, &G.cap_y, O * K * 2)) return 1;
    /* the exact integer decode is bitwise for every code; the host-pointer
     * path is PCIe-bound, so it always takes it */
    HIPCHK(ghip_launch_dequant((const uint8_t *)dc, (const float *)ds,
                               (uint16_t *)G.d_y, O, K, 1, G.stream));
    G.dispatches++;
    return sync_out(out, G.d_y, O * K * 2);
}

/* Hooks: the floors of c/backend_gmetal.mm:437-474, then the direct path. */
static int hook_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                          size_t M, size_t O, size_t K) {
    if (!G.enabled) return 1;
    if (G.max_m > 0 && M > (size_t)G.max_m) return 1;
    if (O * K * 2 < G.min_kb * 1024) return 1;
    return apus_ghip_bf16_gemm(w, x, y, M, O, K);
}

static int hook_fp8blk_linear(const uint8_t *codes, const float *scales,
                              const uint16_t *x, uint16_t *y, size_t M,
                              size_t O, size_t K) {
    if (!G.enabled) return 1;
    if (G.max_m > 0 && M > (size_t)G.max_m) return 1;
    if (O * K < G.fp8_min_kb * 1024) return 1;
    return apus_ghip_fp8blk_linear(codes, scales, x, y, M, O, K);
}

/* ------------------------------------------------------------------------ */
/* device-pointer entry points                                              */
/* ------------------------------------------------------------------------ */

static const uint32_t *exact_flag_dev(const uint8_t *codes, size_t n,
                                      int exact, hipStream_t st, int *rc) {
    *rc = 0;
    if (exact == 0) return NULL;
    if (exact > 0) return G.d_flag + 1;        /* set to 1 once, at init */
    if (ghip_launch_fill_u32(G.d_flag, 1, 0u, st) != hipSuccess
        || ghip_launch_nan_scan(codes, n, G.d_flag, st) != hipSuccess) {
        *rc = 1;
        return NULL;
    }
    return G.d_flag;
}

int apus_ghip_fp8blk_linear_dev(const uint8_t *codes, const float *scales,
                                const uint16_t *x, uint16_t *y,
                                size_t M, size_t O, size_t K,
                                int exact, void *stream) {
    if (ghip_init() || check_sizes(M, O, K)) return 1;
    hipStream_t st = (hipStream_t)stream;
    int rc;
    const uint32_t *flag = exact_flag_dev(codes, O * K, exact, st, &rc);
    if (rc) { ghip_seterr("fp8blk_linear_dev: flag setup failed"); return 1; }
    HIPCHK(ghip_launch_fp8_linear(codes, scales, x, y, M, O, K, flag,
                                  G.trace_n >= 2 ? G.trace_ev : NULL, st));
    G.dispatches++;
    return 0;
}

int apus_ghip_stream_hold(void *stream, uint32_t us) {
    if (ghip_init()) return 1;
    if (us > 1000000u) {
        ghip_seterr("stream_hold: %u us is above the 1 s limit", us);
        return 1;
    }
    int khz = 0;
    HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, G.device));
    if (khz <= 0) {
        ghip_seterr("stream_hold: no wall-clock rate");
        return 1;
    }
    HIPCHK(ghip_launch_hold((uint64_t)us * (uint64_t)khz / 1000u, (hipStream_t)stream));
    return 0;
}

void apus_ghip_set_trace_events(void *const *events, int n) {
    G.trace_n = 0;
    if (!events || n <= 0) return;
    if (n > 8) n = 8;
    for (int i = 0; i < n; i++) G.trace_ev[i] = (hipEvent_t)events[i];
    G.trace_n = n;
}

int apus_ghip_fp8blk_dequant_dev(const uint8_t *codes, const float *scales,
                                 uint16_t *out, size_t O, size_t K,
                                 int exact, void *stream) {
    if (ghip_init() || check_sizes(1, O, K)) return 1;
    /* dequant has no device-side selection: auto means exact (bitwise for
     * every code; the fast decode is for callers that know their codes) */
    HIPCHK(ghip_launch_dequant(codes, scales, out, O, K, exact != 0,
                               (hipStream_t)stream));
    G.dispatches++;
    return 0;
}

int apus_ghip_bf16_gemm_dev(const uint16_t *w, const uint16_t *x,
                            uint16_t *y, size_t M, size_t O, size_t K,
                            void *stream) {
    if (ghip_init() || check_sizes(M, O, K)) return 1;
    HIPCHK(ghip_launch_bf16_linear(w, x, y, M, O, K, G.trace_n >= 2 ? G.trace_ev : NULL,
                                   (hipStream_t)stream));
    G.dispatches++;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* HBM expert slab store                                                    */
/* ------------------------------------------------------------------------ */

struct ApusGhipStore {
    int n_experts;
    size_t dim, inter;
    float limit;
    /* host slab layout (c/gcache.h:852-861) */
    size_t h_gw, h_gs, h_uw, h_us, h_dw, h_ds, h_bytes;
    /* device layout: same order, members 256-byte aligned */
    size_t d_gw, d_gs, d_uw, d_us, d_dw, d_ds, d_stride;
    uint8_t *arena;                      /* n_experts + 1 slabs (the last: shared) */
    uint32_t *nan_flags;                 /* device [n_experts + 1] */
    int has_shared;                      /* the shared slab is set */
    GhipMoeDecodeWs ws;
    /* decode staging for the host-pointer entry */
    uint16_t *d_x, *d_out;
    int32_t *d_idx;
    float *d_w;
};

static size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

int apus_ghip_store_open(ApusGhipStore **out, int n_experts, size_t dim,
                         size_t inter, float limit, char *err, size_t errcap) {
    *out = NULL;
    if (ghip_init()) {
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return 1;
    }
    if (n_experts <= 0 || dim == 0 || inter == 0) {
        ghip_seterr("store_open: bad shape E=%d dim=%zu inter=%zu", n_experts,
                    dim, inter);
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return 1;
    }
    ApusGhipStore *s = (ApusGhipStore *)calloc(1, sizeof *s);
    if (!s) return 1;
    s->n_experts = n_experts;
    s->dim = dim;
    s->inter = inter;
    s->limit = limit;
    size_t nbg = ((inter + 127) / 128) * ((dim + 127) / 128) * sizeof(float);
    size_t nbd = ((dim + 127) / 128) * ((inter + 127) / 128) * sizeof(float);
    s->h_gw = 0;
    s->h_gs = inter * dim;
    s->h_uw = s->h_gs + nbg;
    s->h_us = s->h_uw + inter * dim;
    s->h_dw = s->h_us + nbg;
    s->h_ds = s->h_dw + dim * inter;
    s->h_bytes = s->h_ds + nbd;
    s->d_gw = 0;
    s->d_gs = up256(inter * dim);
    s->d_uw = s->d_gs + up256(nbg);
    s->d_us = s->d_uw + up256(inter * dim);
    s->d_dw = s->d_us + up256(nbg);
    s->d_ds = s->d_dw + up256(dim * inter);
    s->d_stride = s->d_ds + up256(nbd);
    /* one slab more than the routed experts: the shared expert's (set by
     * apus_ghip_store_put_shared) */
    size_t total = s->d_stride * ((size_t)n_experts + 1);
    hipError_t e = hipMalloc((void **)&s->arena, total);
    if (e != hipSuccess) {
        ghip_seterr("store_open: hipMalloc(%zu) %s", total, hipGetErrorString(e));
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        free(s);
        return 1;
    }
    int bad = hipMalloc((void **)&s->nan_flags, ((size_t)n_experts + 1) * 4) != hipSuccess
           || hipMemset(s->nan_flags, 0, ((size_t)n_experts + 1) * 4) != hipSuccess
           || hipMalloc((void **)&s->ws.hw, GHIP_HW_SLOTS * inter * 4) != hipSuccess
           /* both h buffers start as the sentinel (every byte 0xff) */
           || hipMemset(s->ws.hw, 0xff, GHIP_HW_SLOTS * inter * 4) != hipSuccess
           || (s->ws.hw_inter = (uint32_t)inter) == 0
           || hipMalloc((void **)&s->ws.err, 4) != hipSuccess
           || hipMemset(s->ws.err, 0, 4) != hipSuccess
           || hipMalloc((void **)&s->ws.lw, 512 * sizeof(uint64_t)) != hipSuccess
           || hipMemset(s->ws.lw, 0, 512 * sizeof(uint64_t)) != hipSuccess
           || (s->ws.n_cu = G.n_cu_dev) == 0
           || hipMalloc((void **)&s->d_x, dim * 2) != hipSuccess
           || hipMalloc((void **)&s->d_out, dim * 2) != hipSuccess
           || hipMalloc((void **)&s->d_idx, GHIP_MAX_TOPK * 4) != hipSuccess
           || hipMalloc((void **)&s->d_w, GHIP_MAX_TOPK * 4) != hipSuccess;
    if (bad) {
        ghip_seterr("store_open: workspace allocation failed");
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        apus_ghip_store_close(s);
        return 1;
    }
    *out = s;
    return 0;
}

void apus_ghip_store_close(ApusGhipStore *s) {
    if (!s) return;
    hipDeviceSynchronize();
    hipFree(s->arena);
    hipFree(s->nan_flags);
    hipFree(s->ws.hw);
    hipFree(s->ws.err);
    hipFree(s->ws.lw);
    hipFree(s->d_x);
    hipFree(s->d_out);
    hipFree(s->d_idx);
    hipFree(s->d_w);
    free(s);
}

size_t apus_ghip_store_slab_bytes(const ApusGhipStore *s) {
    return s ? s->h_bytes : 0;
}

const void *apus_ghip_store_slab_dev(const ApusGhipStore *s, int expert) {
    if (!s || expert < 0 || expert >= s->n_experts) return NULL;
    return s->arena + (size_t)expert * s->d_stride;
}

/* NaN-code scan of an expert's three code members into nan_flags[e]. */
static int store_scan(ApusGhipStore *s, int e, hipStream_t st) {
    uint8_t *b = s->arena + (size_t)e * s->d_stride;
    uint32_t *f = s->nan_flags + e;
    HIPCHK(ghip_launch_fill_u32(f, 1, 0u, st));
    HIPCHK(ghip_launch_nan_scan(b + s->d_gw, s->inter * s->dim, f, st));
    HIPCHK(ghip_launch_nan_scan(b + s->d_uw, s->inter * s->dim, f, st));
    HIPCHK(ghip_launch_nan_scan(b + s->d_dw, s->dim * s->inter, f, st));
    return 0;
}

static int store_upload(ApusGhipStore *s, int expert, const void *slab);

int apus_ghip_store_put(ApusGhipStore *s, int expert, const void *slab,
                        size_t nbytes) {
    if (!s || expert < 0 || expert >= s->n_experts || nbytes != s->h_bytes) {
        ghip_seterr("store_put: bad expert %d or slab size %zu (want %zu)",
                    expert, nbytes, s ? s->h_bytes : 0);
        return 1;
    }
    return store_upload(s, expert, slab);
}

int apus_ghip_store_put_shared(ApusGhipStore *s, const void *slab, size_t nbytes) {
    if (!s) {
        ghip_seterr("store_put_shared: no store");
        return 1;
    }
    if (!slab) {                         /* remove: routed experts only */
        HIPCHK(hipStreamSynchronize(G.stream));
        s->has_shared = 0;
        return 0;
    }
    if (nbytes != s->h_bytes) {
        ghip_seterr("store_put_shared: slab size %zu (want %zu: the shared expert's "
                    "intermediate must be the store's)", nbytes, s->h_bytes);
        return 1;
    }
    if (store_upload(s, s->n_experts, slab)) return 1;
    s->has_shared = 1;
    return 0;
}

/* One H2D copy of a host slab into arena slot `expert` (n_experts = the
 * shared expert's) and its NaN-code scan. */
static int store_upload(ApusGhipStore *s, int expert, const void *slab) {
    uint8_t *b = s->arena + (size_t)expert * s->d_stride;
    const uint8_t *h = (const uint8_t *)slab;
    int same = s->d_gs == s->h_gs && s->d_uw == s->h_uw && s->d_us == s->h_us
            && s->d_dw == s->h_dw && s->d_ds == s->h_ds;
    if (same) {
        HIPCHK(hipMemcpyAsync(b, h, s->h_bytes, hipMemcpyHostToDevice, G.stream));
    } else {
        const size_t hs[6] = { s->h_gw, s->h_gs, s->h_uw, s->h_us, s->h_dw, s->h_ds };
        const size_t ds[6] = { s->d_gw, s->d_gs, s->d_uw, s->d_us, s->d_dw, s->d_ds };
        for (int i = 0; i < 6; i++) {
            size_t len = (i < 5 ? hs[i + 1] : s->h_bytes) - hs[i];
            HIPCHK(hipMemcpyAsync(b + ds[i], h + hs[i], len,
                                  hipMemcpyHostToDevice, G.stream));
        }
    }
    G.h2d += s->h_bytes;
    if (store_scan(s, expert, G.stream)) return 1;
    HIPCHK(hipStreamSynchronize(G.stream));
    return 0;
}

int apus_ghip_store_get(ApusGhipStore *s, int expert, void *slab, size_t nbytes) {
    if (!s || expert < 0 || expert >= s->n_experts || nbytes != s->h_bytes) {
        ghip_seterr("store_get: bad expert %d or slab size %zu (want %zu)",
                    expert, nbytes, s ? s->h_bytes : 0);
        return 1;
    }
    /* each member from its 256-byte aligned device offset to its host
     * (packed) offset: the inverse of apus_ghip_store_put */
    const uint8_t *b = s->arena + (size_t)expert * s->d_stride;
    uint8_t *h = (uint8_t *)slab;
    const size_t hs[7] = { s->h_gw, s->h_gs, s->h_uw, s->h_us, s->h_dw, s->h_ds, s->h_bytes };
    const size_t ds[6] = { s->d_gw, s->d_gs, s->d_uw, s->d_us, s->d_dw, s->d_ds };
    for (int i = 0; i < 6; i++)
        HIPCHK(hipMemcpyAsync(h + hs[i], b + ds[i], hs[i + 1] - hs[i],
                              hipMemcpyDeviceToHost, G.stream));
    HIPCHK(hipStreamSynchronize(G.stream));
    G.d2h += s->h_bytes;
    return 0;
}

/* Parallel pread of one slab for the container loader. A shard in the host
 * page cache is read at one thread's memcpy rate (~25 GB/s), below the host
 * link, so each slab is split into one part per reader of a pool that
 * lives for one load call; the main thread hands out a slab by posting
 * each reader's semaphore and waits for as many completions. */
#define GHIP_LOAD_THREADS 4

typedef struct {
    sem_t go[GHIP_LOAD_THREADS], done;
    int fd, quit, nthr;
    uint8_t *dst;
    uint64_t off;
    size_t bytes;
    int ok[GHIP_LOAD_THREADS];
} SlabReader;

typedef struct {
    SlabReader *r;
    int t;
} SlabReaderArg;

static int pread_full(int fd, uint8_t *dst, size_t n, uint64_t off) {
    size_t got = 0;
    while (got < n) {
        ssize_t k = pread(fd, dst + got, n - got, (off_t)(off + got));
        if (k <= 0) return 0;
        got += (size_t)k;
    }
    return 1;
}

static void *slab_reader_main(void *arg) {
    SlabReaderArg *a = (SlabReaderArg *)arg;
    SlabReader *r = a->r;
    for (;;) {
        while (sem_wait(&r->go[a->t]) != 0) {}
        if (r->quit) break;
        const size_t part = (r->bytes + (size_t)r->nthr - 1) / (size_t)r->nthr;
        const size_t lo = (size_t)a->t * part < r->bytes ? (size_t)a->t * part : r->bytes;
        const size_t hi = lo + part < r->bytes ? lo + part : r->bytes;
        r->ok[a->t] = pread_full(r->fd, r->dst + lo, hi - lo, r->off + lo);
        sem_post(&r->done);
    }
    return NULL;
}

/* one slab through the pool (nthr > 0) or on this thread */
static int slab_read(SlabReader *r, int fd, uint8_t *dst, size_t n, uint64_t off) {
    if (!r->nthr) return pread_full(fd, dst, n, off);
    r->fd = fd;
    r->dst = dst;
    r->off = off;
    r->bytes = n;
    for (int t = 0; t < r->nthr; t++) sem_post(&r->go[t]);
    int ok = 1;
    for (int t = 0; t < r->nthr; t++) {
        while (sem_wait(&r->done) != 0) {}
    }
    for (int t = 0; t < r->nthr; t++) ok &= r->ok[t];
    return ok;
}

int apus_ghip_store_load_container(ApusGhipStore *s, const char *dir, int layer,
                                   int *n_loaded, char *err, size_t errcap) {
    if (n_loaded) *n_loaded = 0;
    if (err && errcap) err[0] = 0;
    if (!s) {
        ghip_seterr("store_load_container: no store");
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return 1;
    }
    GhipSlabRec *recs = NULL;
    int n = 0;
    char lerr[512] = {0};
    if (ghip_container_layer(dir, layer, s->h_bytes, &recs, &n, lerr, sizeof lerr)) {
        ghip_seterr("%s", lerr);
        if (err && errcap) snprintf(err, errcap, "%s", g_err);
        return 1;
    }
    for (int i = 0; i < n; i++)
        if (recs[i].expert < 0 || recs[i].expert >= s->n_experts) {
            ghip_seterr("store_load_container: record (layers.%d, %d) past the store's %d "
                        "experts", layer, recs[i].expert, s->n_experts);
            if (err && errcap) snprintf(err, errcap, "%s", g_err);
            free(recs);
            return 1;
        }
    /* two pinned slab buffers: the read of slab i+1 overlaps the H2D of
     * slab i (one slab per read, as the reference's one pread per slab,
     * c/gcache.h:394-451, here split over the reader pool) */
    uint8_t *pin[2] = {NULL, NULL};
    hipEvent_t done[2] = {NULL, NULL};
    int fds_n = 0, rc = 0;
    struct { char name[256]; int fd; } fds[64];
    for (int b = 0; b < 2 && !rc; b++)
        rc = hipHostMalloc((void **)&pin[b], s->h_bytes, 0) != hipSuccess
             || hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess;
    if (rc) ghip_seterr("store_load_container: pinned staging (%zu B) failed", s->h_bytes);
    /* reader pool (as many readers as could be started; none: this thread
     * reads) */
    SlabReader rd;
    SlabReaderArg rarg[GHIP_LOAD_THREADS];
    pthread_t rthr[GHIP_LOAD_THREADS];
    memset(&rd, 0, sizeof rd);
    int sems = 0;
    if (sem_init(&rd.done, 0, 0) == 0) {
        sems = 1;
        for (; sems <= GHIP_LOAD_THREADS && sem_init(&rd.go[sems - 1], 0, 0) == 0; sems++) {}
    }
    /* sems - 1 go-semaphores exist */
    for (int t = 0; !rc && t < sems - 1; t++) {
        rarg[t].r = &rd;
        rarg[t].t = t;
        if (pthread_create(&rthr[t], NULL, slab_reader_main, &rarg[t])) break;
        rd.nthr = t + 1;
    }
    int loaded = 0;
    for (int i = 0; i < n && !rc; i++) {
        int fd = -1;
        for (int k = 0; k < fds_n; k++)
            if (!strcmp(fds[k].name, recs[i].shard)) fd = fds[k].fd;
        if (fd < 0) {
            char path[4400];
            snprintf(path, sizeof path, "%s/%s", dir, recs[i].shard);
            fd = open(path, O_RDONLY | O_CLOEXEC);
            if (fd < 0 || fds_n == 64) {
                ghip_seterr("store_load_container: cannot open shard %s", path);
                if (fd >= 0) close(fd);
                rc = 1;
                break;
            }
            snprintf(fds[fds_n].name, sizeof fds[fds_n].name, "%s", recs[i].shard);
            fds[fds_n++].fd = fd;
        }
        uint8_t *h = pin[i & 1];
        if (i >= 2 && hipEventSynchronize(done[i & 1]) != hipSuccess) {
            ghip_seterr("store_load_container: copy failed");
            rc = 1;
            break;
        }
        if (!slab_read(&rd, fd, h, s->h_bytes, recs[i].offset)) {
            ghip_seterr("store_load_container: short read of (layers.%d, %d) in %s",
                        layer, recs[i].expert, recs[i].shard);
            rc = 1;
            break;
        }
        uint8_t *b = s->arena + (size_t)recs[i].expert * s->d_stride;
        const size_t hs[7] = { s->h_gw, s->h_gs, s->h_uw, s->h_us, s->h_dw, s->h_ds,
                               s->h_bytes };
        const size_t ds[6] = { s->d_gw, s->d_gs, s->d_uw, s->d_us, s->d_dw, s->d_ds };
        for (int m = 0; m < 6 && !rc; m++)
            rc = hipMemcpyAsync(b + ds[m], h + hs[m], hs[m + 1] - hs[m],
                                hipMemcpyHostToDevice, G.stream) != hipSuccess;
        if (!rc) rc = store_scan(s, recs[i].expert, G.stream);
        if (!rc) rc = hipEventRecord(done[i & 1], G.stream) != hipSuccess;
        if (rc) {
            ghip_seterr("store_load_container: upload of expert %d failed", recs[i].expert);
            break;
        }
        G.h2d += s->h_bytes;
        loaded++;
    }
    if (hipStreamSynchronize(G.stream) != hipSuccess && !rc) {
        ghip_seterr("store_load_container: sync failed");
        rc = 1;
    }
    rd.quit = 1;
    for (int t = 0; t < rd.nthr; t++) sem_post(&rd.go[t]);
    for (int t = 0; t < rd.nthr; t++) pthread_join(rthr[t], NULL);
    for (int t = 0; t < sems - 1; t++) sem_destroy(&rd.go[t]);
    if (sems) sem_destroy(&rd.done);
    for (int k = 0; k < fds_n; k++) close(fds[k].fd);
    for (int b = 0; b < 2; b++) {
        if (pin[b]) hipHostFree(pin[b]);
        if (done[b]) hipEventDestroy(done[b]);
    }
    free(recs);
    if (n_loaded) *n_loaded = loaded;
    if (rc && err && errcap) snprintf(err, errcap, "%s", g_err);
    return rc;
}

int apus_ghip_store_synth(ApusGhipStore *s, uint64_t seed, int bank,
                          float scale_lo, float scale_hi) {
    if (!s) return 1;
    size_t nbg = ((s->inter + 127) / 128) * ((s->dim + 127) / 128);
    size_t nbd = ((s->dim + 127) / 128) * ((s->inter + 127) / 128);
    size_t nmax = nbg > nbd ? nbg : nbd;
    float *hs = (float *)malloc(nmax * sizeof(float));
    if (!hs) { ghip_seterr("store_synth: out of host memory"); return 1; }
    int rc = 0;
    for (int e = 0; e < s->n_experts && !rc; e++) {
        uint8_t *b = s->arena + (size_t)e * s->d_stride;
        const size_t cw[3] = { s->d_gw, s->d_uw, s->d_dw };
        const size_t cs[3] = { s->d_gs, s->d_us, s->d_ds };
        const size_t ns[3] = { nbg, nbg, nbd };
        for (int j = 0; j < 3 && !rc; j++) {
            uint64_t kc = apus_synth_key(seed, apus_synth_expert_stream(bank, e, 2 * j));
            if (ghip_launch_synth_codes(b + cw[j], s->inter * s->dim, kc, 0,
                                        G.stream) != hipSuccess) {
                ghip_seterr("store_synth: code fill launch failed");
                rc = 1;
                break;
            }
            apus_synth_scales(hs, ns[j], seed,
                              apus_synth_expert_stream(bank, e, 2 * j + 1),
                              scale_lo, scale_hi);
            if (hipMemcpyAsync(b + cs[j], hs, ns[j] * sizeof(float),
                               hipMemcpyHostToDevice, G.stream) != hipSuccess
                || hipStreamSynchronize(G.stream) != hipSuccess) {
                ghip_seterr("store_synth: scale upload failed");
                rc = 1;
            }
        }
        /* synthetic codes exclude 0x7F/0xFF by construction */
        if (!rc && ghip_launch_fill_u32(s->nan_flags + e, 1, 0u, G.stream) != hipSuccess)
            rc = 1;
    }
    free(hs);
    if (!rc && hipStreamSynchronize(G.stream) != hipSuccess) {
        ghip_seterr("store_synth: sync failed");
        rc = 1;
    }
    return rc;
}

int apus_ghip_store_expert_bf16(ApusGhipStore *s, int expert,
                                uint16_t *payload) {
    if (!s || expert < 0 || expert >= s->n_experts) {
        ghip_seterr("store_expert_bf16: bad expert %d", expert);
        return 1;
    }
    size_t n = s->inter * s->dim;
    if (grow(&G.d_y, &G.cap_y, 3 * n * 2)) return 1;
    const uint8_t *b = s->arena + (size_t)expert * s->d_stride;
    uint16_t *o = (uint16_t *)G.d_y;
    HIPCHK(ghip_launch_dequant(b + s->d_gw, (const float *)(b + s->d_gs), o,
                               s->inter, s->dim, 1, G.stream));
    HIPCHK(ghip_launch_dequant(b + s->d_uw, (const float *)(b + s->d_us), o + n,
                               s->inter, s->dim, 1, G.stream));
    HIPCHK(ghip_launch_dequant(b + s->d_dw, (const float *)(b + s->d_ds),
                               o + 2 * n, s->dim, s->inter, 1, G.stream));
    G.dispatches += 3;
    return sync_out(payload, G.d_y, 3 * n * 2);
}

static void store_bank(const ApusGhipStore *s, GhipBank *bk) {
    bk->base = s->arena;
    bk->stride = s->d_stride;
    bk->off_gw = s->d_gw;
    bk->off_gs = s->d_gs;
    bk->off_uw = s->d_uw;
    bk->off_us = s->d_us;
    bk->off_dw = s->d_dw;
    bk->off_ds = s->d_ds;
    bk->n_experts = (uint32_t)s->n_experts;
    bk->dim = (uint32_t)s->dim;
    bk->inter = (uint32_t)s->inter;
    bk->nan_flags = s->nan_flags;
    bk->err = s->ws.err;
    bk->has_shared = (uint32_t)s->has_shared;
}

int apus_ghip_store_status(ApusGhipStore *s, void *stream, int clear,
                           uint32_t *code) {
    if (!s || !code) {
        ghip_seterr("store_status: no store or no code pointer");
        return 1;
    }
    HIPCHK(hipStreamSynchronize((hipStream_t)stream));
    uint32_t v = 0;
    HIPCHK(hipMemcpy(&v, s->ws.err, 4, hipMemcpyDeviceToHost));
    if (clear && v) HIPCHK(hipMemset(s->ws.err, 0, 4));
    *code = v;
    return 0;
}

/* The host-pointer MoE entries report only their own launch's failure: the
 * sticky word is cleared on their stream before they launch. */
static int store_status_clear(ApusGhipStore *s) {
    HIPCHK(hipMemsetAsync(s->ws.err, 0, 4, G.stream));
    return 0;
}

/* ------------------------------------------------------------------------ */
/* synthetic device fills (include/apus_synth.h)                            */
/* ------------------------------------------------------------------------ */

static uint16_t *g_dtab;

int apus_synth_fp8_codes_dev(uint8_t *out, size_t n, uint64_t seed,
                             uint64_t sstream, uint64_t offset, void *stream) {
    if (ghip_init()) return 1;
    HIPCHK(ghip_launch_synth_codes(out, n, apus_synth_key(seed, sstream), offset,
                                   (hipStream_t)stream));
    return 0;
}

int apus_synth_bf16_normal_dev(uint16_t *out, size_t n, uint64_t seed,
                               uint64_t sstream, uint64_t offset, void *stream) {
    if (ghip_init()) return 1;
    if (!g_dtab) {
        HIPCHK(hipMalloc((void **)&g_dtab, 65536 * 2));
        HIPCHK(hipMemcpy(g_dtab, apus_synth_normal_table_ptr(), 65536 * 2,
                         hipMemcpyHostToDevice));
    }
    HIPCHK(ghip_launch_synth_bf16(out, n, apus_synth_key(seed, sstream), offset,
                                  g_dtab, (hipStream_t)stream));
    return 0;
}

int apus_ghip_moe_decode_dev(ApusGhipStore *s, const uint16_t *x,
                             const float *logits, const int32_t *idx,
                             const float *w, int topk, uint16_t *out,
                             void *stream) {
    if (!s) { ghip_seterr("moe_decode: no store"); return 1; }
    if (topk <= 0 || topk > GHIP_MAX_TOPK || topk > s->n_experts) {
        ghip_seterr("moe_decode: topk %d outside 1..%d", topk, GHIP_MAX_TOPK);
        return 1;
    }
    if (!logits && (!idx || !w)) {
        ghip_seterr("moe_decode: need logits or idx+w");
        return 1;
    }
    GhipBank bk;
    store_bank(s, &bk);
    hipError_t e = ghip_launch_moe_decode(&bk, x, logits, idx, w, NULL, topk,
                                          s->limit, out, &s->ws,
                                          G.trace_n >= 2 ? G.trace_ev : NULL,
                                          (hipStream_t)stream);
    if (e != hipSuccess) {
        ghip_seterr("moe_decode launch: %s", hipGetErrorString(e));
        return 1;
    }
    G.dispatches++;
    return 0;
}

int apus_ghip_moe_decode_router_dev(ApusGhipStore *s, const uint16_t *x,
                                    const uint16_t *gate_w, const float *gate_bias,
                                    float route_scale, int topk, uint16_t *out,
                                    int32_t *idx_out, float *w_out, void *stream) {
    if (!s) { ghip_seterr("moe_decode_router: no store"); return 1; }
    if (topk <= 0 || topk > GHIP_MAX_TOPK || topk > s->n_experts || s->n_experts > 512
        || !gate_w || !gate_bias || (!idx_out) != (!w_out)) {
        ghip_seterr("moe_decode_router: bad arguments (E=%d topk=%d; gate_w and bias "
                    "required, idx_out and w_out both or neither, E <= 512)",
                    s->n_experts, topk);
        return 1;
    }
    GhipBank bk;
    store_bank(s, &bk);
    GhipRouterArgs ra = {gate_w, gate_bias, route_scale, idx_out, w_out};
    hipError_t e = ghip_launch_moe_decode(&bk, x, NULL, NULL, NULL, &ra, topk, s->limit,
                                          out, &s->ws,
                                          G.trace_n >= 2 ? G.trace_ev : NULL,
                                          (hipStream_t)stream);
    if (e != hipSuccess) {
        ghip_seterr("moe_decode_router launch: %s (16-byte x / gate_w; E <= 8 x CUs)",
                    hipGetErrorString(e));
        return 1;
    }
    G.dispatches++;
    return 0;
}

/* device router workspace: logits [512] f32, then the one-launch router's
 * arrival counter (one u32, 0 between launches) */
static float *g_router_logits;
#define GHIP_ROUTER_WS_WORDS (512 + 64)

int apus_ghip_moe_router_dev(const uint16_t *x, const uint16_t *gate_w,
                             const float *logits, const float *gate_bias, int E,
                             size_t dim, int topk, float route_scale, float *scores,
                             int32_t *idx, float *w, void *stream) {
    if (ghip_init()) return 1;
    if (E <= 0 || E > 512 || topk <= 0 || topk > GHIP_MAX_TOPK || topk > E
        || !gate_bias || !idx || !w || (!logits && (!x || !gate_w || dim == 0))) {
        ghip_seterr("moe_router: bad arguments (E=%d topk=%d dim=%zu)", E, topk, dim);
        return 1;
    }
    if (!logits && !g_router_logits) {
        HIPCHK(hipMalloc((void **)&g_router_logits, GHIP_ROUTER_WS_WORDS * sizeof(float)));
        HIPCHK(hipMemset(g_router_logits, 0, GHIP_ROUTER_WS_WORDS * sizeof(float)));
        HIPCHK(hipDeviceSynchronize());
    }
    hipError_t e = ghip_launch_moe_router(x, gate_w, logits, g_router_logits,
                                          logits ? NULL : (uint32_t *)(g_router_logits + 512),
                                          gate_bias, (uint32_t)E, (uint32_t)dim, topk,
                                          route_scale, scores, idx, w,
                                          G.trace_n >= 2 ? G.trace_ev : NULL,
                                          (hipStream_t)stream);
    if (e != hipSuccess) {
        ghip_seterr("moe_router launch: %s (dim %% 8 and 16-byte x / gate_w required)",
                    hipGetErrorString(e));
        return 1;
    }
    G.dispatches++;
    return 0;
}

int apus_ghip_moe_decode(ApusGhipStore *s, const uint16_t *x,
                         const int32_t *idx, const float *w, int topk,
                         uint16_t *out) {
    if (!s) { ghip_seterr("moe_decode: no store"); return 1; }
    if (topk <= 0 || topk > GHIP_MAX_TOPK) {
        ghip_seterr("moe_decode: topk %d outside 1..%d", topk, GHIP_MAX_TOPK);
        return 1;
    }
    for (int j = 0; j < topk; j++)
        if (idx[j] < 0 || idx[j] >= s->n_experts) {
            ghip_seterr("moe_decode: expert id %d out of range", idx[j]);
            return 1;
        }
    if (h2d(s->d_x, x, s->dim * 2) || h2d(s->d_idx, idx, (size_t)topk * 4)
        || h2d(s->d_w, w, (size_t)topk * 4))
        return 1;
    if (store_status_clear(s)) return 1;
    if (apus_ghip_moe_decode_dev(s, s->d_x, NULL, s->d_idx, s->d_w, topk,
                                 s->d_out, G.stream))
        return 1;
    if (sync_out(out, s->d_out, s->dim * 2)) return 1;
    uint32_t err = 0;
    if (apus_ghip_store_status(s, G.stream, 1, &err)) return 1;
    if (err) {
        ghip_seterr(err & 4u ? "moe_decode: the gate/up -> down hand-off wait ran out "
                               "(code %u)"
                             : "moe_decode: invalid expert id in routing (code %u)", err);
        return 1;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* K4: routed MoE prefill                                                   */
/* ------------------------------------------------------------------------ */

/* Grow one prefill workspace buffer; the caller has drained the device. */
static int pf_grow(void **p, size_t *cap, size_t need) {
    if (need <= *cap) return 0;
    need = (need + 4095) & ~(size_t)4095;
    if (*p) HIPCHK(hipFree(*p));
    *p = NULL;
    *cap = 0;
    HIPCHK(hipMalloc(p, need));
    *cap = need;
    return 0;
}

int apus_ghip_moe_prefill_reserve(const ApusGhipStore *s, size_t tokens,
                                  int topk) {
    if (ghip_init()) return 1;
    if (!s || topk <= 0 || topk > GHIP_MAX_TOPK) {
        ghip_seterr("moe_prefill_reserve: bad store or topk %d", topk);
        return 1;
    }
    if (!G.pf_inited) {
        HIPCHK(ghip_moe_prefill_init());
        G.pf.n_cu = G.n_cu;
        G.pf_inited = 1;
    }
    /* a shared expert adds one pair per token (and one expert) */
    const size_t P = tokens * ((size_t)topk + (s->has_shared ? 1 : 0));
    if (P == 0) return 0;
    const uint32_t E = (uint32_t)s->n_experts + (s->has_shared ? 1u : 0u);
    _Static_assert(PF_HDR_Q + 16 <= PF_HDR_WORDS, "prefill header holds the queues");
    const size_t need[8] = {
        PF_HDR_WORDS * sizeof(uint32_t),
        ghip_moe_prefill_chunks(P) * E * sizeof(uint32_t),
        ghip_moe_prefill_max_tiles(P, E) * 4 * sizeof(uint32_t),
        P * sizeof(int32_t), P * sizeof(int32_t), P * sizeof(int32_t),
        P * s->inter * 2, P * s->dim * 2};
    int grow_any = 0;
    for (int i = 0; i < 8; i++) grow_any |= need[i] > G.pf_cap[i];
    if (grow_any) {
        HIPCHK(hipDeviceSynchronize());
        void **bufs[8] = {(void **)&G.pf.hdr, (void **)&G.pf.cnt,
                          (void **)&G.pf.tiles, (void **)&G.pf.eid,
                          (void **)&G.pf.perm, (void **)&G.pf.pos,
                          (void **)&G.pf.h, (void **)&G.pf.o};
        for (int i = 0; i < 8; i++)
            if (pf_grow(bufs[i], &G.pf_cap[i], need[i])) return 1;
    }
    /* every buffer now holds this shape's P pairs (the chunk and tile
     * arrays depend on P and E, so the limit is per call, not a max) */
    G.pf.cap_pairs = P;
    return 0;
}

int apus_ghip_moe_prefill_dev(ApusGhipStore *s, const uint16_t *x, size_t T,
                              const int32_t *idx, const float *w, int topk,
                              uint16_t *out, void *stream) {
    if (!s) { ghip_seterr("moe_prefill: no store"); return 1; }
    if (topk <= 0 || topk > GHIP_MAX_TOPK) {
        ghip_seterr("moe_prefill: topk %d outside 1..%d", topk, GHIP_MAX_TOPK);
        return 1;
    }
    if (T == 0) return 0;
    if (s->dim % 256 || s->inter % 128 || s->n_experts + s->has_shared > 1024) {
        ghip_seterr("moe_prefill: needs dim %% 256 == 0, inter %% 128 == 0 and "
                    "<= 1024 experts (dim=%zu inter=%zu E=%d)", s->dim, s->inter,
                    s->n_experts);
        return 1;
    }
    if (apus_ghip_moe_prefill_reserve(s, T, topk)) return 1;
    GhipBank bk;
    store_bank(s, &bk);
    hipError_t e = ghip_launch_moe_prefill(&bk, x, T, idx, w, topk, s->limit, out,
                                           &G.pf,
                                           G.trace_n >= 8 ? G.trace_ev : NULL,
                                           (hipStream_t)stream);
    if (e != hipSuccess) {
        ghip_seterr("moe_prefill launch: %s", hipGetErrorString(e));
        return 1;
    }
    G.dispatches++;
    return 0;
}

int apus_ghip_moe_prefill_dev_noalloc(ApusGhipStore *s, const uint16_t *x, size_t T,
                                      const int32_t *idx, const float *w, int topk,
                                      uint16_t *out, void *stream) {
    /* no allocation and no init here: the store exists, so the library's
     * init (device, kernel attributes, the scratch address) already ran */
    if (!s || !G.inited) {
        ghip_seterr("moe_prefill_noalloc: %s", s ? "library not initialised" : "no store");
        return 1;
    }
    if (topk <= 0 || topk > GHIP_MAX_TOPK) {
        ghip_seterr("moe_prefill_noalloc: topk %d outside 1..%d", topk, GHIP_MAX_TOPK);
        return 1;
    }
    if (T == 0) return 0;
    if (s->dim % 256 || s->inter % 128 || s->n_experts + s->has_shared > 1024) {
        ghip_seterr("moe_prefill_noalloc: needs dim %% 256 == 0, inter %% 128 == 0 and "
                    "<= 1024 experts (dim=%zu inter=%zu E=%d)", s->dim, s->inter,
                    s->n_experts);
        return 1;
    }
    const size_t P = T * ((size_t)topk + (s->has_shared ? 1 : 0));
    const uint32_t Ep = (uint32_t)s->n_experts + (s->has_shared ? 1u : 0u);
    const size_t need = ghip_pf_scratch_need(P, Ep, (uint32_t)s->dim,
                                             (uint32_t)s->inter);
    if (need > GHIP_PF_SCRATCH_BYTES) {
        ghip_seterr("moe_prefill_noalloc: %zu tokens x top-%d need %zu bytes of workspace, "
                    "above the fixed %zu-byte scratch (use apus_ghip_moe_prefill_dev)",
                    T, topk, need, (size_t)GHIP_PF_SCRATCH_BYTES);
        return 1;
    }
    GhipMoePrefillWs ws;
    hipError_t e = ghip_pf_scratch_ws(G.device, P, Ep, (uint32_t)s->dim,
                                      (uint32_t)s->inter, G.n_cu, &ws);
    if (e != hipSuccess) {
        ghip_seterr("moe_prefill_noalloc: scratch: %s", hipGetErrorString(e));
        return 1;
    }
    GhipBank bk;
    store_bank(s, &bk);
    e = ghip_launch_moe_prefill(&bk, x, T, idx, w, topk, s->limit, out, &ws,
                                G.trace_n >= 8 ? G.trace_ev : NULL, (hipStream_t)stream);
    if (e != hipSuccess) {
        ghip_seterr("moe_prefill_noalloc launch: %s", hipGetErrorString(e));
        return 1;
    }
    G.dispatches++;
    return 0;
}

int apus_ghip_moe_prefill(ApusGhipStore *s, const uint16_t *x, size_t T,
                          const int32_t *idx, const float *w, int topk,
                          uint16_t *out) {
    if (!s) { ghip_seterr("moe_prefill: no store"); return 1; }
    if (topk <= 0 || topk > GHIP_MAX_TOPK) {
        ghip_seterr("moe_prefill: topk %d outside 1..%d", topk, GHIP_MAX_TOPK);
        return 1;
    }
    if (T == 0) return 0;
    const size_t P = T * (size_t)topk;
    for (size_t p = 0; p < P; p++)
        if (idx[p] < 0 || idx[p] >= s->n_experts) {
            ghip_seterr("moe_prefill: expert id %d out of range (pair %zu)",
                        idx[p], p);
            return 1;
        }
    if (grow(&G.pf_x, &G.pf_cap_x, T * s->dim * 2)
        || grow(&G.pf_idx, &G.pf_cap_idx, P * 4)
        || grow(&G.pf_w, &G.pf_cap_w, P * 4)
        || grow(&G.pf_out, &G.pf_cap_out, T * s->dim * 2))
        return 1;
    if (h2d(G.pf_x, x, T * s->dim * 2) || h2d(G.pf_idx, idx, P * 4)
        || h2d(G.pf_w, w, P * 4))
        return 1;
    if (store_status_clear(s)) return 1;
    if (apus_ghip_moe_prefill_dev(s, (const uint16_t *)G.pf_x, T,
                                  (const int32_t *)G.pf_idx, (const float *)G.pf_w,
                                  topk, (uint16_t *)G.pf_out, G.stream))
        return 1;
    if (sync_out(out, G.pf_out, T * s->dim * 2)) return 1;
    uint32_t hdr[PF_HDR_WORDS], err = 0;
    HIPCHK(hipMemcpy(hdr, G.pf.hdr, sizeof hdr, hipMemcpyDeviceToHost));
    if (apus_ghip_store_status(s, G.stream, 1, &err)) return 1;
    if (hdr[PF_HDR_ERR] || err) {
        ghip_seterr("moe_prefill: invalid expert id in routing");
        return 1;
    }
    return 0;
}
