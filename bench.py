#!/usr/bin/env python3
"""bench.py — MI355X throughput of the apus FP8-block MoE hot path.

Default workload = BASELINE.json config 2, the metric's "FP8 MoE decode GEMV":
one routed-MoE decode step per launch (288-expert FP8 bank resident in HBM,
one token, device top-8 of f32 logits + softmax, SwiGLU experts, ordered
bf16 combine). Inputs rotate over R tokens/routings so every step streams
8 experts' weights from HBM. value = algorithmic bytes per step (8 expert
slabs + x + out + logits = 201,393,280 B) / measured time, in GB/s.

The default run also carries, in the same line, the dense GEMV configs
("dense": config 0, W [2048,4096], and config 1, W [16384,4096], at
M = 1, 2, 4, over rotating weight copies >= 3x the 256 MB MALL) and the
prefill half of the metric ("prefill": configs 4 and 3). Every object has
its roofline, its CPU leg, the step against both rooflines and the
weight-only GB/s of the reference benches.

--workload dense_gemv / dense_gemv_c0 run config 1 / 0 alone (--m for M);
timed regions measure back-to-back device steps, not Python's launch rate:
after a warmup long enough for the device to settle, the host stays ahead of
the device (a step of 12 us or more against ~3 us per launch), and only config
0's 4.5 us steps start behind a long lead of unrelated device work. --workload dense_gemm runs
the four DSA FP8 projections at M = 2048 prefill rows (the fp8blk_linear
hook's MFMA GEMM path), in TFLOP/s. --workload bf16_gemv runs the LM head
through the bf16_gemm hook; --workload moe_decode_router runs config 2 routed
by the reference's sigmoid/bias router on the GPU; --workload store_load
fills the HBM expert store from a converted v2 container; --workload
library_gemm times the vendor library (torch -> hipBLASLt, BF16) on the
prefill shapes, a practical MFMA reference rather than this build.

Prints ONE JSON line (rank 0). Extra objects: "roofline" (dominant kernel,
HIP-event timed on its stream) and "cpu_baseline" (the reference CPU path,
compiled from the reference sources into oracle/_ref, timed on this host on
a bounded sample; the C restatement in oracle/ when that is absent).
"""
import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "apus-glm5.3-flash_amd")
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, AMD published
BF16_PEAK_TFLOPS = 2500.0        # MI355X dense BF16 MFMA, AMD published
HOST_LINK_PEAK_GBS = 64.0        # PCIe 5.0 x16, one direction (host -> MI355X)


def _cpu_threads():
    """Threads for the CPU baseline: the CPUs this process may run on,
    capped at 16 (the GPU box's CPU share per GPU, whatever nproc shows)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


CPU_THREADS = _cpu_threads()


def cpu_common(O, use_ref):
    """cores (the threads the timed CPU path actually ran on: the reference
    pool's count, which APUS_THREADS sets, c/pool.h:95-104) and the host
    facts of cpu_info()."""
    cores = O.ref().ref_pool_threads() if use_ref else CPU_THREADS
    return {"cores": int(cores), **cpu_info()}


def cpu_info():
    """Host facts the CPU baseline is quoted with: model, nproc, the CPUs
    this process may use and the threads the baseline used."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = None
    return {"cpu_model": model, "host_nproc": os.cpu_count(), "affinity_cpus": aff,
            "threads": CPU_THREADS}


def load_pkg():
    spec = importlib.util.spec_from_file_location(
        "apus_ghip", os.path.join(PKG, "__init__.py"),
        submodule_search_locations=[PKG])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["apus_ghip"] = mod
    spec.loader.exec_module(mod)
    import apus_ghip.hiprt as rt  # noqa: E402
    return mod, rt


def traffic_from_profiles(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration) and committed under
    profiles/; None when no measurement exists for this kernel."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    v = d.get(kernel)
    return v.get("hbm_bytes_per_launch") if isinstance(v, dict) else None


_LIB = None


def lead(st, us=2000):
    """Hold st for `us` microseconds just before the timed region's start
    event (apus_ghip_stream_hold: one wave waiting on the wall clock, no
    memory traffic), so Python has enqueued the timed steps before the
    device reaches them: the timed span is then the device's back-to-back
    step time, not the host's launch rate (steps of a few to tens of
    microseconds)."""
    rc = _LIB.apus_ghip_stream_hold(st.vp, us)
    if rc:
        raise RuntimeError("apus_ghip_stream_hold: %s" % _LIB.apus_ghip_last_error())


def long_lead(steps):
    """A lead long enough for the host to enqueue every timed step before
    the device reaches the first (for steps not much longer than a launch)."""
    return min(20000, max(2000, 15 * steps))


def timed(rt, st, step, first, steps, lead_us=300):
    """Events around exactly `steps` steps enqueued back to back on st
    (after a synchronize and a lead, see lead()); ms per step. The default
    lead is a short head start: when a step takes several host launches'
    time the host stays ahead by itself, and a long idle hold before the
    timed steps measurably slows them (the device leaves its steady state:
    a 20 ms hold cost 0.4-0.8 us per decode step and 0.5 us per config-1
    step). Steps close to the launch time pass long_lead(steps)."""
    st.synchronize()
    rt.synchronize()
    lead(st, lead_us)
    e0, e1 = rt.Event(), rt.Event()
    e0.record(st)
    for i in range(steps):
        step(first + i)
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_ms(e1) / steps


def kernel_times(lib, rt, step, first, steps, n_ev, pairs):
    """Average duration (ms) of chosen launches, from start/stop HIP events
    carried by the launches' own dispatch packets on the launch stream
    (apus_ghip_set_trace_events), over a second pass of `steps` steps right
    after the timed region.
    pairs: {name: (i, j)} -> mean elapsed(events[i], events[j])."""
    evs = [[rt.Event() for _ in range(n_ev)] for _ in range(steps)]
    arr_t = ctypes.c_void_p * n_ev
    for i in range(steps):
        arr = arr_t(*[e.handle for e in evs[i]])
        lib.apus_ghip_set_trace_events(arr, n_ev)
        step(first + i)
    lib.apus_ghip_set_trace_events(None, 0)
    rt.synchronize()
    return {name: sum(evs[i][a].elapsed_ms(evs[i][b]) for i in range(steps)) / steps
            for name, (a, b) in pairs.items()}


def store_errors(lib, store):
    """The store's sticky device error word (apus_ghip_store_status: 2 = an
    expert id was dropped, 4 = a decode hand-off wait ran out), read and
    cleared after the timed work; 0 = every timed step ran in full."""
    code = ctypes.c_uint32(0xFFFFFFFF)
    rc = lib.apus_ghip_store_status(store, None, 1, ctypes.byref(code))
    if rc:
        raise RuntimeError("apus_ghip_store_status: %s" % lib.apus_ghip_last_error())
    return int(code.value)


def verify(r, cpu):
    """The bench object's "verified" record: the device error words of the
    timed work, and the output one step produced (outside the timed region)
    against the reference CPU path's output for the same inputs, which the
    cpu_baseline leg computes while it is timed (the leg's own check; None
    without a CPU leg). Tolerance of tests/tolerance.py."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from tolerance import compare_combined, ULP_FRAC_MIN, REL_MAX
    v = {"device_errors": r.get("_device_errors", 0), "output": None}
    ok = v["device_errors"] == 0
    ref = (cpu or {}).get("_ref_out")
    if ref is not None and r.get("_gpu_out") is not None:
        st = compare_combined(r["_gpu_out"], ref["out"], ref["floor"])
        good = st["frac_le1ulp_scaled"] >= ULP_FRAC_MIN and st["max_rel"] <= REL_MAX
        v["output"] = {"against": ref["what"], "n": st["n"],
                       "frac_le1ulp": round(st["frac_le1ulp"], 6),
                       "frac_le1ulp_scaled": round(st["frac_le1ulp_scaled"], 6),
                       "max_rel": round(st["max_rel"], 6), "ok": bool(good)}
        ok = ok and good
    v["ok"] = bool(ok)
    return v


# --------------------------------------------------------------------------
# config 2: MoE decode
# --------------------------------------------------------------------------

MOE = dict(E=288, k=8, dim=4096, inter=2048, seed=0xC2, limit=10.0)


def moe_algorithmic_bytes(E, k, dim, inter):
    """(step bytes, step flops, gate/up launch bytes). Step: k expert slabs
    (FP8 codes + F32 block scales) + x + out + logits. Gate/up launch (it also
    routes): the k gate and up members + x + logits + the k*inter BF16 h
    rows it writes."""
    nb = lambda n: (n + 127) // 128  # noqa: E731
    gu = 2 * (inter * dim + nb(inter) * nb(dim) * 4)
    slab = gu + dim * inter + nb(dim) * nb(inter) * 4
    return (k * slab + dim * 2 + dim * 2 + E * 4, 2 * k * 3 * inter * dim,
            k * gu + dim * 2 + E * 4 + k * inter * 2)


def synth_slab(lib, seed, bank, e, dim, inter):
    """Host slab of expert e of `bank` from the shared generator (the
    streams apus_ghip_store_synth uses; e = E gives the shared expert's)."""
    nb = lambda n: (n + 127) // 128  # noqa: E731
    parts = []
    for j, (o, kk) in enumerate([(inter, dim), (inter, dim), (dim, inter)]):
        c = np.empty(o * kk, np.uint8)
        lib.apus_synth_fp8_codes(c.ctypes.data_as(ctypes.c_void_p), c.size, seed,
                                 lib.apus_synth_expert_stream(bank, e, 2 * j), 0)
        sc = np.empty(nb(o) * nb(kk), np.float32)
        lib.apus_synth_scales(sc.ctypes.data_as(ctypes.c_void_p), sc.size, seed,
                              lib.apus_synth_expert_stream(bank, e, 2 * j + 1),
                              ctypes.c_float(1e-4), ctypes.c_float(1e-2))
        parts += [c, sc.view(np.uint8)]
    return np.concatenate(parts)


def bench_moe_decode(lib, pkg, rt, steps, warmup, rotate=64, shared=False):
    """Config 2 (one token, 8 routed experts of the 288-expert bank, device
    top-8 + softmax of f32 logits); with shared=True the layer's shared
    expert (c/gmoe.h:325-336) is added last, as every GLM-5.3-Flash MoE
    layer has one (reference/config.json: n_shared_experts 1)."""
    E, k, dim, inter, seed = (MOE[x] for x in ("E", "k", "dim", "inter", "seed"))
    store = ctypes.c_void_p()
    err = ctypes.create_string_buffer(256)
    pkg.check(lib.apus_ghip_store_open(ctypes.byref(store), E, dim, inter,
                                       MOE["limit"], err, 256), "store_open")
    pkg.check(lib.apus_ghip_store_synth(store, seed, 0, 1e-4, 1e-2), "store_synth")
    if shared:
        sl = synth_slab(lib, seed, 0, E, dim, inter)
        pkg.check(lib.apus_ghip_store_put_shared(store, sl.ctypes.data_as(ctypes.c_void_p),
                                                 sl.nbytes), "store_put_shared")
    logits = np.empty((rotate, E), np.float32)
    lib.apus_synth_f32_normal(logits.ctypes.data_as(ctypes.c_void_p), logits.size,
                              seed, 30, 0)
    xs = np.empty((rotate, dim), np.uint16)
    lib.apus_synth_bf16_normal(xs.ctypes.data_as(ctypes.c_void_p), xs.size, seed,
                               31, 0)
    d_log = rt.DevBuf.of(logits)
    d_x = rt.DevBuf.of(xs)
    d_out = rt.DevBuf(rotate * dim * 2)
    st = rt.Stream()

    def step(i):
        j = i % rotate
        rc = lib.apus_ghip_moe_decode_dev(
            store, ctypes.c_void_p(d_x.ptr + j * dim * 2),
            ctypes.c_void_p(d_log.ptr + j * E * 4), None, None, k,
            ctypes.c_void_p(d_out.ptr + j * dim * 2), st.vp)
        if rc:
            pkg.check(rc, "moe_decode_dev")

    for i in range(warmup):
        step(i)
    t0 = time.perf_counter()
    ms = timed(rt, st, step, warmup, steps)
    wall = time.perf_counter() - t0
    kt = kernel_times(lib, rt, step, warmup + steps, steps, 2, {"k_moe_decode": (0, 1)})
    # checks outside the timed region: no step lost its work on the device,
    # and rotation 0's output (every step of it writes the same bits)
    errors = store_errors(lib, store)
    out0 = d_out.download(np.uint16, (rotate, dim))[0]
    nbytes, flops, _ = moe_algorithmic_bytes(E, k + (1 if shared else 0), dim, inter)
    gbs = nbytes / (ms * 1e-3) / 1e9
    lib.apus_ghip_store_close(store)
    # the step is one launch: routing, gate/up, hand-off, down + combine
    kern = {"kernel": "k_moe_decode", "kernel_ms": kt["k_moe_decode"],
            "kernel_bytes": nbytes, "kernel_flops": flops,
            "launch_ms": {n: round(v, 5) for n, v in kt.items()}}
    cfg = {"workload": "moe_decode (BASELINE config 2)", "experts": E,
           "topk": k, "dim": dim, "inter": inter, "tokens": 1,
           "rotated_tokens": rotate, "weights": "fp8-e4m3 128x128 blocks",
           "routing": "device top-8 of f32 logits, softmax"}
    if shared:
        cfg["workload"] = ("moe_decode_shared (BASELINE config 2 + the layer's shared "
                           "expert, c/gmoe.h:325-336)")
        cfg["shared_experts"] = 1
    return {
        "ms_per_step": ms, "value": gbs, "wall_s": wall, "one_launch_per_step": True,
        "_device_errors": errors, "_gpu_out": out0,
        "weight_bytes": (k + (1 if shared else 0)) * 3 * inter * dim,
        "bytes": nbytes, "flops": flops, **kern,
        "traffic_key": "k_moe_decode@shared" if shared else "k_moe_decode",
        "config": cfg,
    }


def cpu_moe_decode(lib, budget_s=12.0, shared=False):
    """Reference CPU path for config 2 on this host: per token, the 8
    routed experts (c/gmoe.h:210-227 on BF16 payloads, dequantized on fill as
    c/gcache.h:413-426) and the ordered combine (c/gmoe.h:307-320). The
    dequant-on-fill is timed separately. Bounded sample: tokens until the
    budget is spent."""
    os.environ.setdefault("APUS_THREADS", str(CPU_THREADS))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    E, k, dim, inter, seed = (MOE[x] for x in ("E", "k", "dim", "inter", "seed"))
    use_ref = O.ref_available()
    P = O.ptr
    logits = np.empty(E, np.float32)
    lib.apus_synth_f32_normal(P(logits), E, seed, 30, 0)
    idx, w = O.route_softmax(logits, k)
    payloads, t_deq = [], 0.0
    for e in sorted(int(v) for v in idx):
        mats = []
        for j, (o, kk) in enumerate([(inter, dim), (inter, dim), (dim, inter)]):
            c = np.empty((o, kk), np.uint8)
            lib.apus_synth_fp8_codes(P(c), c.size, seed,
                                     lib.apus_synth_expert_stream(0, e, 2 * j), 0)
            s = np.empty((O.nblocks(o), O.nblocks(kk)), np.float32)
            lib.apus_synth_scales(P(s), s.size, seed,
                                  lib.apus_synth_expert_stream(0, e, 2 * j + 1),
                                  1e-4, 1e-2)
            out = np.empty((o, kk), np.uint16)
            t0 = time.perf_counter()
            if use_ref:
                O.ref().ref_fp8blk_dequant_mt(P(c), P(s), P(out), o, kk)
            else:
                O.lib().apo_fp8blk_dequant_mt(P(c), P(s), P(out), o, kk, CPU_THREADS)
            t_deq += time.perf_counter() - t0
            mats.append(out)
        payloads.append((e, mats))
    if shared:
        # the shared expert's payload (dequantized at open by the reference,
        # c/gmodel.h:962-997; timed with the fills), added after the routed sum
        mats = []
        for j, (o, kk) in enumerate([(inter, dim), (inter, dim), (dim, inter)]):
            c = np.empty((o, kk), np.uint8)
            lib.apus_synth_fp8_codes(P(c), c.size, seed,
                                     lib.apus_synth_expert_stream(0, E, 2 * j), 0)
            sc_ = np.empty((O.nblocks(o), O.nblocks(kk)), np.float32)
            lib.apus_synth_scales(P(sc_), sc_.size, seed,
                                  lib.apus_synth_expert_stream(0, E, 2 * j + 1), 1e-4, 1e-2)
            out = np.empty((o, kk), np.uint16)
            t0 = time.perf_counter()
            if use_ref:
                O.ref().ref_fp8blk_dequant_mt(P(c), P(sc_), P(out), o, kk)
            else:
                O.lib().apo_fp8blk_dequant_mt(P(c), P(sc_), P(out), o, kk, CPU_THREADS)
            t_deq += time.perf_counter() - t0
            mats.append(out)
        shared_pl = mats
    wsorted = {int(i): float(v) for i, v in zip(idx, w)}
    x = np.empty(dim, np.uint16)
    ntok, t_tok = 0, 0.0
    eo = np.empty(dim, np.uint16)
    ref_out, floor = None, np.zeros(dim)
    while t_tok < budget_s and ntok < 4000:
        lib.apus_synth_bf16_normal(P(x), dim, seed, 31, ntok * dim)
        t0 = time.perf_counter()
        y = np.zeros(dim, np.float32)
        for e, (g, u, d) in payloads:
            if use_ref:
                O.ref().ref_gmoe_expert(P(g), P(u), P(d), P(x), dim, inter,
                                        MOE["limit"], P(eo))
            else:
                eo[:] = O.swiglu_expert(g, u, d, x, threads=CPU_THREADS)[0]
            c = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo) * np.float32(wsorted[e])))
            y = O.bf16_to_f32(O.f32_to_bf16(y + c))
            if ntok == 0:
                floor += np.abs(c.astype(np.float64))
        if shared:
            g, u, d = shared_pl
            if use_ref:
                O.ref().ref_gmoe_expert(P(g), P(u), P(d), P(x), dim, inter,
                                        MOE["limit"], P(eo))
            else:
                eo[:] = O.swiglu_expert(g, u, d, x, threads=CPU_THREADS)[0]
            y = O.bf16_to_f32(O.f32_to_bf16(y + O.bf16_to_f32(eo)))   # c/gmoe.h:325-336
            if ntok == 0:
                floor += np.abs(O.bf16_to_f32(eo).astype(np.float64))
        t_tok += time.perf_counter() - t0
        if ntok == 0:
            ref_out = O.f32_to_bf16(y)         # the bench's rotation 0 (x, logits)
        ntok += 1
    nbytes = moe_algorithmic_bytes(E, k + (1 if shared else 0), dim, inter)[0]
    per_tok = t_tok / ntok
    return {
        "value": nbytes / per_tok / 1e9, "unit": "GB/s",
        **cpu_common(O, use_ref),
        "kind": "reference" if use_ref else "port",
        "sample": ("%d decode tokens x %d experts on pre-dequantized BF16 payloads "
                   "(%.1f ms/token); dequant-on-fill of those experts %.1f ms "
                   "reported separately, not in value"
                   % (ntok, k + (1 if shared else 0), per_tok * 1e3, t_deq * 1e3)),
        "ms_per_token": per_tok * 1e3, "dequant_fill_ms": t_deq * 1e3,
        "_ref_out": {"out": ref_out, "floor": floor,
                     "what": "token 0: the reference's expert calls + combine"},
    }


# --------------------------------------------------------------------------
# config 1: dense FP8 GEMV at M = 1, 2, 4
# --------------------------------------------------------------------------

DENSE = {0: dict(N=2048, K=4096, seed=0xC0, copies=92),
         1: dict(N=16384, K=4096, seed=0xC1, copies=12)}


def bench_dense_gemv(lib, pkg, rt, steps, warmup, M=1, cfg=1):
    """BASELINE config 0 (W [2048, 4096]) or 1 (W [16384, 4096]) at M rows:
    one apus_ghip_fp8blk_linear_dev call per step, rotating over weight
    copies that together span >= 3x the 256 MB MALL (92 x 8.4 MB, 12 x 67
    MB), so every step reads its weights from HBM."""
    N, K, seed, copies = (DENSE[cfg][k] for k in ("N", "K", "seed", "copies"))
    nsb = (N // 128) * (K // 128)
    codes = rt.DevBuf(copies * N * K)
    for c in range(copies):
        pkg.check(lib.apus_synth_fp8_codes_dev(ctypes.c_void_p(codes.ptr + c * N * K),
                                               N * K, seed + c, 10, 0, None),
                  "synth codes")
    sc = np.empty((copies, nsb), np.float32)
    for c in range(copies):
        lib.apus_synth_scales(sc[c].ctypes.data_as(ctypes.c_void_p), nsb, seed + c,
                              11, 1e-4, 1e-2)
    d_s = rt.DevBuf.of(sc)
    x = np.empty((M, K), np.uint16)
    lib.apus_synth_bf16_normal(x.ctypes.data_as(ctypes.c_void_p), x.size, seed, 12, 0)
    d_x = rt.DevBuf.of(x)
    d_y = rt.DevBuf(M * N * 2)
    st = rt.Stream()

    def step(i):
        c = i % copies
        rc = lib.apus_ghip_fp8blk_linear_dev(
            ctypes.c_void_p(codes.ptr + c * N * K),
            ctypes.c_void_p(d_s.ptr + c * nsb * 4), d_x.vp, d_y.vp, M, N, K, 0, st.vp)
        if rc:
            pkg.check(rc, "fp8blk_linear_dev")

    for i in range(warmup):
        step(i)
    # config 0's 4.5 us steps are close to a launch's host time: all of them
    # are enqueued behind a long lead before the device starts them
    ms = timed(rt, st, step, warmup, steps,
               lead_us=long_lead(steps) if cfg == 0 else 300)
    kt = kernel_times(lib, rt, step, warmup + steps, steps, 2,
                      {"k_fp8_gemv": (0, 1)})
    step(0)                        # weight copy 0, the CPU leg's inputs (untimed)
    st.synchronize()
    y0 = d_y.download(np.uint16, (M, N))
    nbytes = N * K + nsb * 4 + M * K * 2 + M * N * 2
    return {"ms_per_step": ms, "value": nbytes / (ms * 1e-3) / 1e9,
            "one_launch_per_step": True, "_gpu_out": y0,
            "weight_bytes": N * K, "traffic_key": "k_fp8_gemv@config%d_M%d" % (cfg, M),
            "bytes": nbytes, "flops": 2 * M * N * K, "kernel": "k_fp8_gemv",
            "kernel_ms": kt["k_fp8_gemv"], "kernel_bytes": nbytes,
            "kernel_flops": 2 * M * N * K,
            "launch_ms": {n: round(v, 5) for n, v in kt.items()},
            "config": {"workload": "dense_gemv%s (BASELINE config %d)"
                                   % ("_c0" if cfg == 0 else "", cfg), "N": N, "K": K,
                       "M": M, "weight_copies": copies}}


def cpu_dense_gemv(lib, M=1, cfg=1, budget_s=10.0):
    """The reference's FP8 linear on the CPU (dequant_mt + gemm_mt,
    c/gdsa.h:532-533) on the config's inputs; also the BF16-only GEMV on
    pre-dequantized weights (the MoE decode path, c/gmoe.h:215-226) and the
    scalar anchor on one thread (c/fp8blk.h:115-136 + c/bf16.h:202-217)."""
    os.environ.setdefault("APUS_THREADS", str(CPU_THREADS))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    N, K, seed = (DENSE[cfg][k] for k in ("N", "K", "seed"))
    P = O.ptr
    codes = np.empty((N, K), np.uint8)
    lib.apus_synth_fp8_codes(P(codes), codes.size, seed, 10, 0)
    sc = np.empty((N // 128, K // 128), np.float32)
    lib.apus_synth_scales(P(sc), sc.size, seed, 11, 1e-4, 1e-2)
    x = np.empty((M, K), np.uint16)
    lib.apus_synth_bf16_normal(P(x), x.size, seed, 12, 0)
    y = np.empty((M, N), np.uint16)
    use_ref = O.ref_available()
    n, t = 0, 0.0
    while t < budget_s and n < 2000:
        t0 = time.perf_counter()
        if use_ref:
            O.ref().ref_fp8blk_linear_mt(P(codes), P(sc), P(x), P(y), M, N, K)
        else:
            O.lib().apo_fp8blk_linear(P(codes), P(sc), P(x), P(y), M, N, K, CPU_THREADS)
        t += time.perf_counter() - t0
        n += 1
    nbytes = N * K + sc.size * 4 + M * K * 2 + M * N * 2
    extra = {}
    if use_ref:
        wb = np.empty((N, K), np.uint16)
        O.ref().ref_fp8blk_dequant_mt(P(codes), P(sc), P(wb), N, K)
        n2, t2 = 0, 0.0
        while t2 < budget_s / 4 and n2 < 2000:
            t0 = time.perf_counter()
            O.ref().ref_bf16_gemm_mt(P(wb), P(x), P(y), M, N, K)
            t2 += time.perf_counter() - t0
            n2 += 1
        extra["bf16_gemv_only"] = {
            "value": (N * K * 2 + M * K * 2 + M * N * 2) / (t2 / n2) / 1e9, "unit": "GB/s",
            "sample": "%d calls of apus_bf16_gemm_mt on pre-dequantized BF16 weights "
                      "(%.2f ms/call)" % (n2, t2 / n2 * 1e3)}
        extra["scalar_anchor"] = scalar_anchor(O, codes, sc, x)
    # the reference output of the timed call and its tolerance floor
    # (2^-8 * sum_k |w * x|, f64 over the bit-exact BF16 weights)
    ref_y = y.copy()
    if use_ref:
        O.ref().ref_fp8blk_linear_mt(P(codes), P(sc), P(x), P(ref_y), M, N, K)
    floor = 2.0 ** -8 * O.absdot(O.dequant(codes, sc, threads=CPU_THREADS), x)
    return {"value": nbytes / (t / n) / 1e9, "unit": "GB/s", **extra,
            **cpu_common(O, use_ref),
            "kind": "reference" if use_ref else "port",
            "sample": "%d calls of dequant_mt + gemm_mt (c/gdsa.h:532-533), "
                      "M=%d, %.1f ms/call" % (n, M, t / n * 1e3),
            "_ref_out": {"out": ref_y, "floor": floor,
                         "what": "weight copy 0: the reference's dequant_mt + gemm_mt"}}


def scalar_anchor(O, codes, sc, x):
    """The reference's scalar anchors on ONE thread (apus_fp8blk_dequant_scalar
    then apus_bf16_gemm_scalar, c/fp8blk.h:115-136, c/bf16.h:202-217) on a
    bounded slice of the weight rows (<= 512), reported per FP8 weight byte
    (GB/s of the slice's algorithmic bytes)."""
    P = O.ptr
    N, K = codes.shape
    M = x.shape[0]
    rows = min(N, 512)
    c = np.ascontiguousarray(codes[:rows])
    s = np.ascontiguousarray(sc[:(rows + 127) // 128])
    wb = np.empty((rows, K), np.uint16)
    y = np.empty((M, rows), np.uint16)
    t0 = time.perf_counter()
    O.ref().ref_fp8blk_dequant_scalar(P(c), P(s), P(wb), rows, K)
    O.ref().ref_bf16_gemm_scalar(P(wb), P(x), P(y), M, rows, K)
    t = time.perf_counter() - t0
    nbytes = rows * K + s.size * 4 + M * K * 2 + M * rows * 2
    return {"value": nbytes / t / 1e9, "unit": "GB/s", "threads": 1,
            "sample": "scalar dequant + scalar GEMM on %d of %d weight rows, M=%d "
                      "(%.1f ms)" % (rows, N, M, t * 1e3)}


# --------------------------------------------------------------------------
# FP8-block linear at prefill M (the fp8blk_linear hook's MFMA GEMM path)
# --------------------------------------------------------------------------

# the DSA projections routed through the hook (c/gdsa.h:599-611,660-661)
DSA_SHAPES = [("q_a", 1536, 4096), ("q_b", 16384, 1536), ("kv_a", 512, 4096),
              ("o_proj", 4096, 16384)]


def bench_dense_gemm(lib, pkg, rt, steps, warmup, M=2048):
    """One step = the four DSA FP8 projections of one layer at M prefill
    rows, each one apus_ghip_fp8blk_linear_dev call (weights resident in
    HBM, one copy per shape). FLOPs = 2*M*N*K summed; the dominant kernel
    (roofline) is o_proj's GEMM launch."""
    seed = 0xD5
    mats = []
    for i, (nm, N, K) in enumerate(DSA_SHAPES):
        nsb = (N // 128) * (K // 128)
        codes = rt.DevBuf(N * K)
        pkg.check(lib.apus_synth_fp8_codes_dev(codes.vp, N * K, seed + i, 10, 0, None),
                  "synth codes")
        sc = np.empty(nsb, np.float32)
        lib.apus_synth_scales(sc.ctypes.data_as(ctypes.c_void_p), nsb, seed + i, 11,
                              1e-4, 1e-2)
        x = rt.DevBuf(M * K * 2)
        pkg.check(lib.apus_synth_bf16_normal_dev(x.vp, M * K, seed + i, 12, 0, None),
                  "synth x")
        mats.append((nm, N, K, codes, rt.DevBuf.of(sc), x, rt.DevBuf(M * N * 2)))
    st = rt.Stream()

    def step(_i):
        for (nm, N, K, codes, d_s, x, y) in mats:
            rc = lib.apus_ghip_fp8blk_linear_dev(codes.vp, d_s.vp, x.vp, y.vp, M, N, K,
                                                 0, st.vp)
            if rc:
                pkg.check(rc, "fp8blk_linear_dev " + nm)

    for i in range(warmup):
        step(i)
    ms = timed(rt, st, step, warmup, steps)
    # per-launch times of each projection (dispatch-packet events)
    per = {}
    for (nm, N, K, codes, d_s, x, y) in mats:
        evs = [[rt.Event() for _ in range(2)] for _ in range(steps)]
        arr_t = ctypes.c_void_p * 2
        for i in range(steps):
            lib.apus_ghip_set_trace_events(arr_t(*[e.handle for e in evs[i]]), 2)
            pkg.check(lib.apus_ghip_fp8blk_linear_dev(codes.vp, d_s.vp, x.vp, y.vp, M, N,
                                                      K, 0, st.vp), "linear")
        lib.apus_ghip_set_trace_events(None, 0)
        rt.synchronize()
        per[nm] = sum(ev[0].elapsed_ms(ev[1]) for ev in evs) / steps
    flops = sum(2 * M * N * K for (_, N, K) in DSA_SHAPES)
    nbytes = sum(N * K + (N // 128) * (K // 128) * 4 + M * K * 2 + M * N * 2
                 for (_, N, K) in DSA_SHAPES)
    No, Ko = DSA_SHAPES[3][1], DSA_SHAPES[3][2]
    return {
        "ms_per_step": ms, "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
        "weight_bytes": sum(N * K for (_n, N, K) in DSA_SHAPES),
        "bytes": nbytes, "flops": flops, "kernel": "k_fp8_gemm",
        "kernel_ms": per["o_proj"], "kernel_flops": 2 * M * No * Ko,
        "kernel_bytes": No * Ko + (No // 128) * (Ko // 128) * 4 + M * Ko * 2 + M * No * 2,
        "traffic_key": "k_fp8_gemm@o_proj",
        "launch_ms": {n_: round(v, 5) for n_, v in per.items()},
        "hbm_gbs": nbytes / (ms * 1e-3) / 1e9,
        "config": {"workload": "dense_gemm (DSA FP8 projections at prefill M, "
                               "c/gdsa.h:599-611,660-661)", "M": M,
                   "shapes": {nm: [N, K] for (nm, N, K) in DSA_SHAPES},
                   "weights": "fp8-e4m3 128x128 blocks"},
    }


def cpu_dense_gemm(lib, M=2048, budget_s=10.0):
    """The reference's FP8 linear at M rows is dequant_mt + gemm_mt
    (c/gdsa.h:532-533): timed on a bounded row sample of q_b and converted to
    TFLOP/s (its cost is linear in M)."""
    os.environ.setdefault("APUS_THREADS", str(CPU_THREADS))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    P = O.ptr
    N, K, Ms = 16384, 1536, 16
    codes = np.empty((N, K), np.uint8)
    lib.apus_synth_fp8_codes(P(codes), codes.size, 0xD5, 10, 0)
    sc = np.empty((N // 128, K // 128), np.float32)
    lib.apus_synth_scales(P(sc), sc.size, 0xD5, 11, 1e-4, 1e-2)
    x = np.empty((Ms, K), np.uint16)
    lib.apus_synth_bf16_normal(P(x), x.size, 0xD5, 12, 0)
    y = np.empty((Ms, N), np.uint16)
    use_ref = O.ref_available()
    n, t = 0, 0.0
    while t < budget_s and n < 200:
        t0 = time.perf_counter()
        if use_ref:
            O.ref().ref_fp8blk_linear_mt(P(codes), P(sc), P(x), P(y), Ms, N, K)
        else:
            O.lib().apo_fp8blk_linear(P(codes), P(sc), P(x), P(y), Ms, N, K, CPU_THREADS)
        t += time.perf_counter() - t0
        n += 1
    tflops = 2 * Ms * N * K / (t / n) / 1e12
    return {"value": tflops, "unit": "TFLOP/s",
            **cpu_common(O, use_ref),
            "kind": "reference" if use_ref else "port",
            "sample": "%d calls of dequant_mt + gemm_mt on q_b [16384, 1536], %d rows, "
                      "%.1f ms/call; %d rows of all four projections would take %.1f s"
                      % (n, Ms, t / n * 1e3, M,
                         sum(2 * M * N_ * K_ for (_, N_, K_) in DSA_SHAPES) / (tflops * 1e12))}


# --------------------------------------------------------------------------
# BF16 GEMV hook at decode: the LM head (c/bf16.h:712-767)
# --------------------------------------------------------------------------

# vocab_size x hidden_size of the reference's model config
LM_HEAD = (154880, 4096)


def bench_bf16_gemv(lib, pkg, rt, steps, warmup, M=1, copies=2):
    """One step = one apus_ghip_bf16_gemm_dev call of the LM head
    ([154880, 4096] BF16, 1.27 GB, larger than the 256 MB MALL; two copies
    alternate). Bytes = weights + x + y."""
    N, K = LM_HEAD
    W = rt.DevBuf(copies * N * K * 2)
    pkg.check(lib.apus_synth_bf16_normal_dev(W.vp, copies * N * K, 0xB1, 1, 0, None),
              "synth w")
    x = rt.DevBuf(M * K * 2)
    pkg.check(lib.apus_synth_bf16_normal_dev(x.vp, M * K, 0xB1, 2, 0, None), "synth x")
    y = rt.DevBuf(M * N * 2)
    st = rt.Stream()

    def step(i):
        rc = lib.apus_ghip_bf16_gemm_dev(ctypes.c_void_p(W.ptr + (i % copies) * N * K * 2),
                                         x.vp, y.vp, M, N, K, st.vp)
        if rc:
            pkg.check(rc, "bf16_gemm_dev")

    for i in range(warmup):
        step(i)
    ms = timed(rt, st, step, warmup, steps)
    kname = "k_fp8_gemv_stream<%d, 2, true>" % min(M, 4)
    kt = kernel_times(lib, rt, step, warmup + steps, steps, 2, {kname: (0, 1)})
    nbytes = N * K * 2 + M * K * 2 + M * N * 2
    return {"ms_per_step": ms, "value": nbytes / (ms * 1e-3) / 1e9,
            "weight_bytes": N * K * 2,
            "bytes": nbytes, "flops": 2 * M * N * K, "kernel": kname,
            "kernel_ms": kt[kname], "kernel_bytes": nbytes,
            "kernel_flops": 2 * M * N * K, "traffic_key": "k_bf16_gemv@lm_head",
            "launch_ms": {n: round(v, 5) for n, v in kt.items()},
            "config": {"workload": "bf16_gemv (LM head through the bf16_gemm hook, "
                                   "c/bf16.h:712-767)", "N": N, "K": K, "M": M,
                       "weight_copies": copies, "weights": "bf16"}}


def cpu_bf16_gemv(lib, M=1, budget_s=10.0):
    """The reference's BF16 GEMV (apus_bf16_gemm_mt, c/bf16.h:444-649) on the
    LM head, timed over a bounded number of calls."""
    os.environ.setdefault("APUS_THREADS", str(CPU_THREADS))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    P = O.ptr
    N, K = LM_HEAD
    w = np.empty((N, K), np.uint16)
    lib.apus_synth_bf16_normal(P(w), w.size, 0xB1, 1, 0)
    x = np.empty((M, K), np.uint16)
    lib.apus_synth_bf16_normal(P(x), x.size, 0xB1, 2, 0)
    y = np.empty((M, N), np.uint16)
    use_ref = O.ref_available()
    n, t = 0, 0.0
    while t < budget_s and n < 200:
        t0 = time.perf_counter()
        if use_ref:
            O.ref().ref_bf16_gemm_mt(P(w), P(x), P(y), M, N, K)
        else:
            O.lib().apo_bf16_gemm_mt(P(w), P(x), P(y), M, N, K, CPU_THREADS)
        t += time.perf_counter() - t0
        n += 1
    nbytes = N * K * 2 + M * K * 2 + M * N * 2
    return {"value": nbytes / (t / n) / 1e9, "unit": "GB/s",
            **cpu_common(O, use_ref),
            "kind": "reference" if use_ref else "port",
            "sample": "%d calls of bf16_gemm_mt on the LM head [%d, %d], M=%d, "
                      "%.1f ms/call" % (n, N, K, M, t / n * 1e3)}


# --------------------------------------------------------------------------
# config 2 with the reference router (sigmoid, selection-only bias)
# --------------------------------------------------------------------------

ROUTE_SCALE = 2.5      # routed_scaling_factor of the reference's model config


def router_inputs(lib, E, dim, seed):
    """gate_w [E, dim] bf16 ~ N(0, 1/dim) (N(0, 1) scaled by 2^-6, exact in
    bf16) and bias [E] ~ 0.05 N(0, 1). With N(0, 1) weights the logits
    against an N(0, 1) x have std 64, the sigmoid saturates at 1.0 for ~40%
    of the experts, and the selection-only bias then picks nearly the same
    experts every token (30 distinct over 64 tokens), served from the MALL
    instead of HBM; trained routers' logits are O(1)."""
    gwh = np.empty(E * dim, np.uint16)
    lib.apus_synth_bf16_normal(gwh.ctypes.data_as(ctypes.c_void_p), gwh.size, seed, 40, 0)
    gwf = (gwh.astype(np.uint32) << 16).view(np.float32) * np.float32(1.0 / 64.0)
    gw = (gwf.view(np.uint32) >> 16).astype(np.uint16).reshape(E, dim)
    bias = np.empty(E, np.float32)
    lib.apus_synth_f32_normal(bias.ctypes.data_as(ctypes.c_void_p), E, seed, 41, 0)
    return gw, (bias * np.float32(0.05)).astype(np.float32)


def bench_moe_decode_router(lib, pkg, rt, steps, warmup, rotate=64):
    """One step = the engine's decode step with the reference router
    (sigmoid, stable top-8 of score + bias, pairwise normalization x 2.5,
    c/gmoe.h:191-208) in ONE launch, apus_ghip_moe_decode_router_dev: the
    gate GEMV over gate_w [288, 4096] BF16, the selection, the 8 experts and
    the combine. The two-launch form (apus_ghip_moe_router_dev, then
    apus_ghip_moe_decode_dev with its picks, on one stream) is timed beside
    it. Bytes = 8 expert slabs + x + out + gate_w + bias."""
    E, k, dim, inter, seed = (MOE[x] for x in ("E", "k", "dim", "inter", "seed"))
    store = ctypes.c_void_p()
    err = ctypes.create_string_buffer(256)
    pkg.check(lib.apus_ghip_store_open(ctypes.byref(store), E, dim, inter,
                                       MOE["limit"], err, 256), "store_open")
    pkg.check(lib.apus_ghip_store_synth(store, seed, 0, 1e-4, 1e-2), "store_synth")
    gwh, bias = router_inputs(lib, E, dim, seed)
    gw = rt.DevBuf.of(gwh)
    d_bias = rt.DevBuf.of(bias)
    xs = np.empty((rotate, dim), np.uint16)
    lib.apus_synth_bf16_normal(xs.ctypes.data_as(ctypes.c_void_p), xs.size, seed, 31, 0)
    d_x = rt.DevBuf.of(xs)
    d_out = rt.DevBuf(rotate * dim * 2)
    d_out2 = rt.DevBuf(rotate * dim * 2)
    d_idx = rt.DevBuf(64 * 4)
    d_w = rt.DevBuf(64 * 4)
    st = rt.Stream()

    def fused(i):
        j = i % rotate
        rc = lib.apus_ghip_moe_decode_router_dev(
            store, ctypes.c_void_p(d_x.ptr + j * dim * 2), gw.vp, d_bias.vp,
            ctypes.c_float(ROUTE_SCALE), k, ctypes.c_void_p(d_out.ptr + j * dim * 2),
            None, None, st.vp)
        if rc:
            pkg.check(rc, "moe_decode_router_dev")

    def router(i):
        j = i % rotate
        rc = lib.apus_ghip_moe_router_dev(ctypes.c_void_p(d_x.ptr + j * dim * 2), gw.vp,
                                          None, d_bias.vp, E, dim, k,
                                          ctypes.c_float(ROUTE_SCALE), None, d_idx.vp,
                                          d_w.vp, st.vp)
        if rc:
            pkg.check(rc, "moe_router_dev")

    def decode(i):
        j = i % rotate
        rc = lib.apus_ghip_moe_decode_dev(store, ctypes.c_void_p(d_x.ptr + j * dim * 2),
                                          None, d_idx.vp, d_w.vp, k,
                                          ctypes.c_void_p(d_out2.ptr + j * dim * 2), st.vp)
        if rc:
            pkg.check(rc, "moe_decode_dev")

    def both(i):
        router(i)
        decode(i)

    for i in range(warmup):
        fused(i)
    ms = timed(rt, st, fused, warmup, steps)
    kt = kernel_times(lib, rt, fused, warmup + steps, steps, 2, {"k_moe_decode": (0, 1)})
    for i in range(warmup):
        both(i)
    ms2 = timed(rt, st, both, warmup, steps)
    errors = store_errors(lib, store)
    out0 = d_out.download(np.uint16, (rotate, dim))[0]
    same = bool(np.array_equal(d_out.download(np.uint16, (rotate, dim)),
                               d_out2.download(np.uint16, (rotate, dim))))
    lib.apus_ghip_store_close(store)
    full, _, _ = moe_algorithmic_bytes(E, k, dim, inter)
    nbytes = full - E * 4 + E * dim * 2 + E * 4         # gate_w + bias, no logits
    return {
        "ms_per_step": ms, "value": nbytes / (ms * 1e-3) / 1e9, "_device_errors": errors,
        "_gpu_out": out0, "one_launch_per_step": True,
        "weight_bytes": k * 3 * inter * dim + E * dim * 2,
        "bytes": nbytes, "flops": 2 * k * 3 * inter * dim + 2 * E * dim,
        "kernel": "k_moe_decode", "kernel_ms": kt["k_moe_decode"], "kernel_bytes": nbytes,
        "kernel_flops": 2 * k * 3 * inter * dim + 2 * E * dim,
        "traffic_key": "k_moe_decode@router",
        "launch_ms": {n_: round(v, 5) for n_, v in kt.items()},
        "two_launch": {"ms_per_step": round(ms2, 6),
                       "value": round(nbytes / (ms2 * 1e-3) / 1e9, 2),
                       "outputs_bitwise_equal_to_one_launch": same},
        "config": {"workload": "moe_decode_router (BASELINE config 2 shapes, routed by "
                               "the reference router in the same launch)", "experts": E,
                   "topk": k, "dim": dim, "inter": inter, "tokens": 1,
                   "rotated_tokens": rotate, "route_scale": ROUTE_SCALE,
                   "weights": "fp8-e4m3 128x128 blocks",
                   "routing": "sigmoid + selection-only bias, pairwise-sum x 2.5"},
    }


def cpu_moe_decode_router(lib, budget_s=3.0):
    """The reference router (apus_gmoe_router, c/gmoe.h:191-208) on this
    host, timed and added to the config-2 expert sample of cpu_moe_decode;
    and, untimed, the reference output of the bench's token 0 (its router
    picks, those experts on BF16 payloads, the combine) for the check."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    P = O.ptr
    E, k, dim, inter, seed = (MOE[x] for x in ("E", "k", "dim", "inter", "seed"))
    gw, bias = router_inputs(lib, E, dim, seed)
    x = np.empty(dim, np.uint16)
    lib.apus_synth_bf16_normal(P(x), dim, seed, 31, 0)
    sc, idx, w = (np.empty(E, np.float32), np.empty(k, np.int32), np.empty(k, np.float32))
    use_ref = O.ref_available()
    n, t = 0, 0.0
    while t < budget_s and n < 5000:
        t0 = time.perf_counter()
        if use_ref:
            O.ref().ref_gmoe_router(P(gw), P(bias), E, dim, k, ROUTE_SCALE, P(x), P(sc),
                                    P(idx), P(w))
        else:
            sc, idx, w = O.gmoe_router(gw, bias, x, k, ROUTE_SCALE)
        t += time.perf_counter() - t0
        n += 1
    experts = cpu_moe_decode(lib)
    per_tok = experts["ms_per_token"] * 1e-3 + t / n
    nbytes = moe_algorithmic_bytes(E, k, dim, inter)[0] - E * 4 + E * dim * 2 + E * 4
    # the check's reference: token 0 through the router's picks
    y = np.zeros(dim, np.float32)
    floor = np.zeros(dim)
    eo = np.empty(dim, np.uint16)
    for e, wt in sorted(zip(idx.tolist(), w.tolist())):
        mats = []
        for j, (o, kk) in enumerate([(inter, dim), (inter, dim), (dim, inter)]):
            c = np.empty((o, kk), np.uint8)
            lib.apus_synth_fp8_codes(P(c), c.size, seed,
                                     lib.apus_synth_expert_stream(0, e, 2 * j), 0)
            s_ = np.empty((O.nblocks(o), O.nblocks(kk)), np.float32)
            lib.apus_synth_scales(P(s_), s_.size, seed,
                                  lib.apus_synth_expert_stream(0, e, 2 * j + 1), 1e-4, 1e-2)
            mats.append(O.dequant(c, s_, threads=CPU_THREADS))
        if use_ref:
            O.ref().ref_gmoe_expert(P(mats[0]), P(mats[1]), P(mats[2]), P(x), dim, inter,
                                    MOE["limit"], P(eo))
        else:
            eo[:] = O.swiglu_expert(*mats, x, threads=CPU_THREADS)[0]
        c_ = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo) * np.float32(wt)))
        y = O.bf16_to_f32(O.f32_to_bf16(y + c_))
        floor += np.abs(c_.astype(np.float64))
    experts.update({
        "value": nbytes / per_tok / 1e9,
        "sample": experts["sample"] + "; router %d calls, %.3f ms/call, added"
                  % (n, t / n * 1e3),
        "router_ms": t / n * 1e3,
        "_ref_out": {"out": O.f32_to_bf16(y), "floor": floor,
                     "what": "token 0: the reference router's picks, experts, combine"}})
    return experts


# --------------------------------------------------------------------------
# HBM expert store filled from a converted v2 container
# --------------------------------------------------------------------------

def write_bench_container(root, layer, n_experts, slab):
    """A converted-v2 container (apus.index.json expert_slabs records
    {block, expert, shard, offset, nbytes}, tests/m1/README.md:21-55) with
    one shard holding n_experts copies of `slab`, each at its own offset."""
    os.makedirs(root, exist_ok=True)
    hdr = json.dumps({"__metadata__": {"format": "pt"}}).encode()
    hdr += b" " * ((8 - len(hdr) % 8) % 8)
    recs = []
    name = "apus-00001.safetensors"
    with open(os.path.join(root, name), "wb") as f:
        f.write(len(hdr).to_bytes(8, "little"))
        f.write(hdr)
        off = 8 + len(hdr)
        for e in range(n_experts):
            f.write(slab)
            recs.append({"block": "layers.%d" % layer, "expert": e, "shard": name,
                         "offset": off, "nbytes": len(slab)})
            off += len(slab)
    with open(os.path.join(root, "apus.index.json"), "w") as f:
        json.dump({"format_version": 2, "model_type": "glm5_next",
                   "expert_slabs": recs}, f)
    return os.path.getsize(os.path.join(root, name))


def bench_store_load(lib, pkg, rt, steps, warmup, n_experts=64):
    """One step = apus_ghip_store_load_container of one layer's n_experts
    slabs (25,171,968 B each at 4096/2048) from a container written just
    before, so the shard is in the host page cache: the rate is pread into
    pinned staging overlapped with the H2D copies, not disk. One slab is
    read back and compared with the file."""
    import tempfile
    E, dim, inter = MOE["E"], MOE["dim"], MOE["inter"]
    store = ctypes.c_void_p()
    err = ctypes.create_string_buffer(512)
    pkg.check(lib.apus_ghip_store_open(ctypes.byref(store), E, dim, inter,
                                       MOE["limit"], err, 512), "store_open")
    sb = lib.apus_ghip_store_slab_bytes(store)
    rng = np.random.default_rng(0x5B)
    slab = rng.integers(0, 256, size=sb, dtype=np.uint8).tobytes()
    layer = 3
    with tempfile.TemporaryDirectory(prefix="apus_bench_") as d:
        fsz = write_bench_container(d, layer, n_experts, slab)
        nl = ctypes.c_int(0)
        times = []
        for i in range(warmup + steps):
            t0 = time.perf_counter()
            rc = lib.apus_ghip_store_load_container(store, d.encode(), layer,
                                                    ctypes.byref(nl), err, 512)
            if rc:
                raise RuntimeError("store_load_container: " + err.value.decode())
            if i >= warmup:
                times.append(time.perf_counter() - t0)
        if nl.value != n_experts:
            raise RuntimeError("loaded %d slabs, expected %d" % (nl.value, n_experts))
        back = np.empty(sb, np.uint8)
        pkg.check(lib.apus_ghip_store_get(store, n_experts - 1,
                                          back.ctypes.data_as(ctypes.c_void_p), sb),
                  "store_get")
        if back.tobytes() != slab:
            raise RuntimeError("slab read back differs from the container bytes")
    lib.apus_ghip_store_close(store)
    ms = sum(times) / len(times) * 1e3
    nbytes = n_experts * sb
    return {"ms_per_step": ms, "value": nbytes / (ms * 1e-3) / 1e9,
            "weight_bytes": nbytes,
            "bytes": nbytes, "flops": 0, "kernel": "store_load_container",
            "kernel_ms": ms, "kernel_bytes": nbytes, "kernel_flops": 0,
            "launch_ms": {"store_load_container": round(ms, 4)},
            "host_link": True,
            "config": {"workload": "store_load (one layer of a converted v2 container "
                                   "-> HBM store, page-cache resident)",
                       "slabs": n_experts, "slab_bytes": sb, "shard_bytes": fsz}}


def cpu_store_load(lib, n_experts=8, budget_s=8.0):
    """The reference's fill of one expert (c/gcache.h:394-451 pread, then the
    dequant-on-fill c/gcache.h:413-426: three fp8blk dequants to BF16) on this
    host, from page-cache-resident slabs, in slab GB/s."""
    import tempfile
    os.environ.setdefault("APUS_THREADS", str(CPU_THREADS))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    P = O.ptr
    dim, inter = MOE["dim"], MOE["inter"]
    nb = O.nblocks
    members = [(inter, dim), (inter, dim), (dim, inter)]
    sizes = []
    for (o, kk) in members:
        sizes += [o * kk, nb(o) * nb(kk) * 4]
    sb = sum(sizes)
    rng = np.random.default_rng(0x5C)
    slab = rng.integers(0, 256, size=sb, dtype=np.uint8)
    # scales: positive finite floats
    off = 0
    for m, sz in enumerate(sizes):
        if m % 2:
            slab[off:off + sz] = np.full(sz // 4, 1e-3, np.float32).view(np.uint8)
        off += sz
    use_ref = O.ref_available()
    with tempfile.TemporaryDirectory(prefix="apus_cpu_") as d:
        path = os.path.join(d, "slabs.bin")
        with open(path, "wb") as f:
            for _ in range(n_experts):
                f.write(slab.tobytes())
        fd = os.open(path, os.O_RDONLY)
        buf = np.empty(sb, np.uint8)
        outs = [np.empty(o * kk, np.uint16) for (o, kk) in members]
        n, t = 0, 0.0
        try:
            while t < budget_s and n < 400:
                t0 = time.perf_counter()
                got = os.preadv(fd, [memoryview(buf)], (n % n_experts) * sb)
                if got != sb:
                    raise RuntimeError("short read")
                off = 0
                for j, (o, kk) in enumerate(members):
                    c = buf[off:off + o * kk]
                    s = buf[off + o * kk:off + o * kk + nb(o) * nb(kk) * 4]
                    if use_ref:
                        O.ref().ref_fp8blk_dequant_mt(P(c), P(s), P(outs[j]), o, kk)
                    else:
                        O.lib().apo_fp8blk_dequant_mt(P(c), P(s), P(outs[j]), o, kk,
                                                      CPU_THREADS)
                    off += o * kk + nb(o) * nb(kk) * 4
                t += time.perf_counter() - t0
                n += 1
        finally:
            os.close(fd)
    return {"value": sb / (t / n) / 1e9, "unit": "GB/s",
            **cpu_common(O, use_ref),
            "kind": "reference" if use_ref else "port",
            "sample": "%d slab fills (pread + dequant-on-fill of the 3 members to BF16), "
                      "%.2f ms/slab" % (n, t / n * 1e3)}


# --------------------------------------------------------------------------
# configs 3 / 4: routed-MoE prefill (grouped GEMM, MFMA path)
# --------------------------------------------------------------------------

PREFILL = {
    # config 3's steps settle over the first ~0.3 s after its bank is filled
    # (5 warmup steps read 1.96-1.98 ms, 150 read 1.94); config 4's 16-layer
    # steps are long enough that more warmup only heats the device
    "prefill_zipf": dict(layers=1, T=2048, zipf=1.1, seed=0xC3, steps=40, warmup=150,
                         desc="BASELINE config 3: 288 experts, T=2048, Zipf(1.1) top-8"),
    "prefill_stack": dict(layers=16, T=8192, zipf=0.0, seed=0xC4, steps=5, warmup=2,
                          desc="BASELINE config 4: 16 layers x 288 experts, "
                               "T=8192 per layer, uniform top-8"),
}


def bench_prefill(lib, pkg, rt, steps, warmup, name):
    """One step = the MoE prefill of every layer back to back (one
    apus_ghip_moe_prefill_dev call per layer, each on its own 288-expert
    bank, tokens and routing). FLOPs = pairs x 2*(2*inter*dim + dim*inter);
    algorithmic bytes = the touched experts' FP8 slabs + x + out + routing."""
    cfg = PREFILL[name]
    E, k, dim, inter = 288, 8, 4096, 2048
    L, T, seed = cfg["layers"], cfg["T"], cfg["seed"]
    err = ctypes.create_string_buffer(256)
    stores, xs, idxs, ws, outs, touched = [], [], [], [], [], []
    slab = moe_algorithmic_bytes(E, 1, dim, inter)[0] - 2 * dim * 2 - E * 4
    for l in range(L):
        st_ = ctypes.c_void_p()
        pkg.check(lib.apus_ghip_store_open(ctypes.byref(st_), E, dim, inter,
                                           MOE["limit"], err, 256), "store_open")
        pkg.check(lib.apus_ghip_store_synth(st_, seed + l, l, 1e-4, 1e-2), "store_synth")
        stores.append(st_)
        idx = np.empty((T, k), np.int32)
        w = np.empty((T, k), np.float32)
        pkg.check(lib.apus_synth_route(idx.ctypes.data_as(ctypes.c_void_p),
                                       w.ctypes.data_as(ctypes.c_void_p), T, E, k,
                                       cfg["zipf"], seed + l), "synth_route")
        touched.append(int(np.unique(idx).size))
        d_x = rt.DevBuf(T * dim * 2)
        pkg.check(lib.apus_synth_bf16_normal_dev(d_x.vp, T * dim, seed + l, 40, 0,
                                                 None), "synth x")
        xs.append(d_x)
        idxs.append(rt.DevBuf.of(idx))
        ws.append(rt.DevBuf.of(w))
        outs.append(rt.DevBuf(T * dim * 2))
    pkg.check(lib.apus_ghip_moe_prefill_reserve(stores[0], T, k), "prefill_reserve")
    st = rt.Stream()
    rt.synchronize()

    def step(_i):
        for l in range(L):
            rc = lib.apus_ghip_moe_prefill_dev(stores[l], xs[l].vp, T, idxs[l].vp,
                                               ws[l].vp, k, outs[l].vp, st.vp)
            if rc:
                pkg.check(rc, "moe_prefill_dev")

    for i in range(warmup):
        step(i)
    ms = timed(rt, st, step, warmup, steps)
    # per-launch timing: 8 dispatch-packet events per layer call
    evs = [[rt.Event() for _ in range(8)] for _ in range(L * steps)]
    arr_t = ctypes.c_void_p * 8
    for i in range(steps):
        for l in range(L):
            lib.apus_ghip_set_trace_events(arr_t(*[e.handle for e in evs[i * L + l]]), 8)
            rc = lib.apus_ghip_moe_prefill_dev(stores[l], xs[l].vp, T, idxs[l].vp,
                                               ws[l].vp, k, outs[l].vp, st.vp)
            if rc:
                pkg.check(rc, "moe_prefill_dev")
    lib.apus_ghip_set_trace_events(None, 0)
    rt.synchronize()
    n = len(evs)
    kt = {nm: sum(ev[a].elapsed_ms(ev[b]) for ev in evs) / n
          for nm, (a, b) in {"k_pf_permute": (0, 1), "k_pf_gemm_gateup": (2, 3),
                             "k_pf_gemm_down": (4, 5), "k_pf_combine": (6, 7)}.items()}
    # checks outside the timed region: the device error words of every
    # layer's store, and layer 0's first rows (the CPU leg's sample)
    errors = 0
    for s_ in stores:
        errors |= store_errors(lib, s_)
    out0 = outs[0].download(np.uint16, (T, dim))[:PREFILL_CPU_TOKENS].copy()
    for s_ in stores:
        lib.apus_ghip_store_close(s_)
    P = T * k
    flops = L * P * 2 * 3 * inter * dim
    nbytes = sum(touched) * slab + L * (2 * T * dim * 2 + P * 8)
    gu_flops = P * 2 * 2 * inter * dim
    # gate/up launch bytes: the touched experts' gate and up members, the
    # gathered x rows (one per pair) and the BF16 h rows it writes
    nb = lambda n: (n + 127) // 128  # noqa: E731
    gu_member = 2 * (inter * dim + nb(inter) * nb(dim) * 4)
    gu_bytes = sum(touched) // L * gu_member + P * dim * 2 + P * inter * 2
    return {
        "ms_per_step": ms, "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
        "_device_errors": errors, "_gpu_out": out0,
        "weight_bytes": sum(touched) * 3 * inter * dim,
        "bytes": nbytes, "flops": flops, "kernel": "k_pf_gemm_gateup",
        "kernel_ms": kt["k_pf_gemm_gateup"], "kernel_flops": gu_flops,
        "kernel_bytes": gu_bytes, "traffic_key": "k_pf_gemm_gateup@" + name,
        # config 3 moves ~113 FLOP per HBM byte, below the ~315 FLOP/B ridge:
        # HBM-bound (config 4, ~447 FLOP/B, is MFMA-bound)
        "bound": "hbm" if cfg["zipf"] > 0 else "mfma",
        "launch_ms": {n_: round(v, 5) for n_, v in kt.items()},
        "hbm_gbs": nbytes / (ms * 1e-3) / 1e9,
        "config": {"workload": "%s (%s)" % (name, cfg["desc"]), "layers": L,
                   "experts": E, "topk": k, "dim": dim, "inter": inter,
                   "tokens_per_layer": T,
                   "routing": "Zipf(%.1f)" % cfg["zipf"] if cfg["zipf"] > 0 else "uniform",
                   "experts_touched_per_layer": touched[0] if L == 1 else
                   [min(touched), max(touched)],
                   "weights": "fp8-e4m3 128x128 blocks"},
    }


def _cpu_prefill_expert(O, P, use_ref, item, idx, x, dim, inter, eo, out, acc):
    """Dequant-on-fill of one expert (timed into acc["deq"]), then its calls
    for every sample token routed to it (timed into acc["exp"])."""
    e, members = item
    mats = []
    for (c, sc) in members:
        o, kk = c.shape
        pl = np.empty((o, kk), np.uint16)
        t0 = time.perf_counter()
        if use_ref:
            O.ref().ref_fp8blk_dequant_mt(P(c), P(sc), P(pl), o, kk)
        else:
            O.lib().apo_fp8blk_dequant_mt(P(c), P(sc), P(pl), o, kk, CPU_THREADS)
        acc["deq"] += time.perf_counter() - t0
        mats.append(pl)
    g, u, d = mats
    if "floor" in acc:
        # untimed: each routed token's expert-output floor sum_i |h_i * wd_i|
        # (the oracle's h), which the check carries through the combine
        toks = np.nonzero((idx == e).any(1))[0]
        slab = np.concatenate([np.ascontiguousarray(a).view(np.uint8).ravel()
                               for cs in members for a in cs])
        bank = [None] * (e + 1)
        bank[e] = slab
        fe = O.moe_expert_floor(bank, dim, inter, x[toks], np.full((len(toks), 1), e,
                                np.int32), np.ones((len(toks), 1), np.float32),
                                limit=MOE["limit"], threads=CPU_THREADS)
        for r, t in enumerate(toks):
            acc["floor"][(int(t), e)] = fe[r]
    for t in np.nonzero((idx == e).any(1))[0]:
        t0 = time.perf_counter()
        if use_ref:
            O.ref().ref_gmoe_expert(P(g), P(u), P(d), P(x[t]), dim, inter, MOE["limit"],
                                    P(out))
        else:
            out[:] = O.swiglu_expert(g, u, d, x[t], threads=CPU_THREADS)[0]
        acc["exp"] += time.perf_counter() - t0
        eo[(int(t), e)] = out.copy()


PREFILL_CPU_TOKENS = 128


def cpu_moe_prefill(lib, name, ntok=PREFILL_CPU_TOKENS):
    """The reference has no grouped GEMM: its prefill is the per-token loop
    (c/gmoe.h:278-320), each token's selected experts (apus_gmoe_expert on
    BF16 payloads, c/gmoe.h:210-227) then the ascending-expert bf16-per-add
    combine (c/gmoe.h:307-320). Timed on a real sample: the first `ntok`
    tokens of the config's first layer with their own routing and inputs
    (the bench's generator streams). The expert calls run expert by expert
    (each expert's payload is dequantized once, then called for each sample
    token routed to it -- the same calls the per-token loop makes); the
    dequant-on-fill is timed apart and not in value. value = TFLOP/s of the
    sample (50,331,648 FLOP per (token, expert)); the full config is
    extrapolated linearly from it."""
    os.environ.setdefault("APUS_THREADS", str(CPU_THREADS))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    P = O.ptr
    cfg = PREFILL[name]
    E, k, dim, inter, seed = 288, 8, 4096, 2048, cfg["seed"]
    T = cfg["T"]
    use_ref = O.ref_available()
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    lib.apus_synth_route(P(idx), P(w), T, E, k, cfg["zipf"], seed)
    idx, w = idx[:ntok].copy(), w[:ntok].copy()
    x = np.empty((ntok, dim), np.uint16)
    lib.apus_synth_bf16_normal(P(x), x.size, seed, 40, 0)
    eo = {}
    out = np.empty(dim, np.uint16)
    shapes = [(inter, dim), (inter, dim), (dim, inter)]

    def gen(e):
        """expert e's FP8 members (untimed; the generator is not the reference)"""
        mm = []
        for j, (o, kk) in enumerate(shapes):
            c = np.empty((o, kk), np.uint8)
            lib.apus_synth_fp8_codes(P(c), c.size, seed,
                                     lib.apus_synth_expert_stream(0, e, 2 * j), 0)
            sc = np.empty((O.nblocks(o), O.nblocks(kk)), np.float32)
            lib.apus_synth_scales(P(sc), sc.size, seed,
                                  lib.apus_synth_expert_stream(0, e, 2 * j + 1), 1e-4, 1e-2)
            mm.append((c, sc))
        return mm

    from concurrent.futures import ThreadPoolExecutor
    experts = sorted(set(idx.ravel().tolist()))
    batches = [experts[i:i + CPU_THREADS] for i in range(0, len(experts), CPU_THREADS)]
    # generation runs in parallel between the timed parts, never beside them
    acc = {"deq": 0.0, "exp": 0.0, "floor": {}}
    with ThreadPoolExecutor(CPU_THREADS) as ex:
        for b in batches:
            for e, members in zip(b, list(ex.map(gen, b))):
                _cpu_prefill_expert(O, P, use_ref, (e, members), idx, x, dim, inter, eo,
                                    out, acc)
    t_deq, t_exp = acc["deq"], acc["exp"]
    t0 = time.perf_counter()
    ref_out = np.empty((ntok, dim), np.uint16)
    for t in range(ntok):
        y = np.zeros(dim, np.float32)
        seen = set()
        for e, wt in sorted(zip(idx[t].tolist(), w[t].tolist())):
            if e in seen:
                continue
            seen.add(e)
            c = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo[(t, e)]) * np.float32(wt)))
            y = O.bf16_to_f32(O.f32_to_bf16(y + c))
        ref_out[t] = O.f32_to_bf16(y)
    t_comb = time.perf_counter() - t0
    # the combine's tolerance floor (untimed): sum_e |contrib_e|, or each
    # expert output's own floor carried through the weights when larger
    floor_c, floor_e = np.zeros((ntok, dim)), np.zeros((ntok, dim))
    for (t, e), o in eo.items():
        wt = w[t][list(idx[t]).index(e)]
        floor_c[t] += np.abs(O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(o) * np.float32(wt)))
                             .astype(np.float64))
        floor_e[t] += abs(float(wt)) * acc["floor"][(t, e)]
    floor = np.maximum(floor_c, floor_e)
    pairs = len(eo)
    tsec = t_exp + t_comb
    full_pairs = cfg["layers"] * T * k
    return {"value": pairs * 50_331_648 / tsec / 1e12, "unit": "TFLOP/s", **cpu_common(O, use_ref),
            "kind": "reference" if use_ref else "port",
            "sample": ("the first %d tokens of layer 0 with their own routing (%d (token, "
                       "expert) pairs over %d distinct experts): expert calls %.2f s + "
                       "combine %.3f s; dequant-on-fill of those experts %.2f s, not in "
                       "value; the full config (%d pairs) extrapolates linearly to %.0f s"
                       % (ntok, pairs, len(set(idx.ravel().tolist())), t_exp, t_comb, t_deq,
                          full_pairs, tsec * full_pairs / pairs)),
            "dequant_fill_s": t_deq,
            "_ref_out": {"out": ref_out, "floor": floor,
                         "what": "layer 0, tokens 0..%d: the reference's per-token loop"
                                 % (ntok - 1)}}


# --------------------------------------------------------------------------
# calibration: a plain device-to-device copy of known size
# --------------------------------------------------------------------------

def bench_copy(rt, steps, warmup, nbytes=256 << 20):
    """hipMemcpyAsync D2D of 256 MiB (the runtime's copy kernel): the
    known-size reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    a, b = rt.DevBuf(nbytes), rt.DevBuf(nbytes)
    a.zero()
    st = rt.Stream()
    h = rt.hip()
    for _ in range(warmup):
        rt.check(h.hipMemcpyAsync(b.vp, a.vp, nbytes, rt.D2D, st.vp), "copy")
    st.synchronize()
    e0, e1 = rt.Event(), rt.Event()
    e0.record(st)
    for _ in range(steps):
        rt.check(h.hipMemcpyAsync(b.vp, a.vp, nbytes, rt.D2D, st.vp), "copy")
    e1.record(st)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    return {"ms_per_step": ms, "value": 2 * nbytes / (ms * 1e-3) / 1e9,
            "bytes": 2 * nbytes, "flops": 0, "kernel": "copy",
            "kernel_ms": ms, "kernel_bytes": 2 * nbytes, "kernel_flops": 0,
            "launch_ms": {"copy": round(ms, 5)},
            "config": {"workload": "copy (FETCH/WRITE calibration)",
                       "bytes_read": nbytes, "bytes_written": nbytes}}


def bench_library_gemm(steps, warmup):
    """The vendor library on the prefill shapes, as a practical MFMA
    reference: torch (hipBLASLt) BF16 x BF16 products with no dequant, no
    gather and no epilogue. Batched: config 4's gate/up and down shapes
    (288 experts x 228 rows, the uniform routing's mean); dense: two large
    GEMMs. Both operands contiguous (batched bf16 products with a
    transposed right operand are avoided on this platform). The first
    shape is the line's value."""
    import torch
    dev = "cuda:0"
    shapes = [("grouped gate/up 288x[228,4096]x[4096,4096]", 288, 228, 4096, 4096),
              ("grouped down 288x[228,2048]x[2048,4096]", 288, 228, 4096, 2048),
              ("dense [65536,4096]x[4096,4096]", 1, 65536, 4096, 4096),
              ("dense [8192,4096]x[4096,4096]", 1, 8192, 4096, 4096)]
    g = torch.Generator(device=dev)
    g.manual_seed(0x11B)
    res = {}
    first = None
    for name, G, M, N, K in shapes:
        a = torch.randn(G, M, K, device=dev, dtype=torch.bfloat16, generator=g)
        b = torch.randn(G, K, N, device=dev, dtype=torch.bfloat16, generator=g)
        fn = (lambda: torch.bmm(a, b)) if G > 1 else (lambda: a[0] @ b[0])
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        flops = 2.0 * G * M * N * K
        res[name] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
        if first is None:
            first = (name, ms, flops)
        del a, b
    name, ms, flops = first
    return {"ms_per_step": ms, "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
            "bytes": 0, "flops": flops, "kernel": "hipBLASLt " + name,
            "kernel_ms": ms, "kernel_bytes": 0, "kernel_flops": flops,
            "launch_ms": {n: v["ms"] for n, v in res.items()},
            "traffic_key": "none", "data": "synthetic (torch.randn, seeded)",
            "config": {"workload": "library_gemm (hipBLASLt via torch, BF16, "
                                   "prefill shapes; a reference, not this build)",
                       "results": res}}


# --------------------------------------------------------------------------

def mfma_busy_from_profiles(key):
    """MFMA-busy fraction of a kernel measured with rocprofv3 --pmc
    (SQ_VALU_MFMA_BUSY_CYCLES over SQ_BUSY_CYCLES x CUs, committed under
    profiles/mfma_busy.json); None when not measured."""
    path = os.path.join(ROOT, "profiles", "mfma_busy.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        v = json.load(f).get(key)
    return v.get("mfma_busy_frac") if isinstance(v, dict) else None


def roofline_of(r):
    key = r.get("traffic_key", r["kernel"])
    traffic = traffic_from_profiles(key)
    src = "dispatch-packet events"
    if r.get("one_launch_per_step") and r["kernel_ms"] > r["ms_per_step"]:
        # one launch per step: the back-to-back step bounds the launch from
        # above; the per-launch events of short launches read longer than the
        # step (they include the packet's own event writes)
        src = ("back-to-back step (the dispatch-packet events read %.6f ms, above "
               "the step)" % r["kernel_ms"])
        r = dict(r, kernel_ms=r["ms_per_step"])
    mfma = r.get("unit") == "TFLOP/s" and r.get("bound", "mfma") == "mfma"
    if mfma:
        achieved = r["kernel_flops"] / (r["kernel_ms"] * 1e-3) / 1e12
    else:
        achieved = r["kernel_bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
    peak = BF16_PEAK_TFLOPS if mfma else HBM_PEAK_GBS
    bound = "mfma" if mfma else "hbm"
    if r.get("host_link"):
        peak, bound = HOST_LINK_PEAK_GBS, "pcie"
    return {
        "bound": bound,
        "kernel": r["kernel"],
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": "TFLOP/s" if mfma else "GB/s",
        "frac": round(achieved / peak, 4),
        "traffic": traffic,
        "algorithmic_bytes_per_launch": r["kernel_bytes"],
        "algorithmic_flops_per_launch": r["kernel_flops"],
        "avg_launch_ms": round(r["kernel_ms"], 6),
        "launch_time_source": src,
        "launch_ms": r["launch_ms"],
        "mfma_tflops": round(r["kernel_flops"] / (r["kernel_ms"] * 1e-3) / 1e12, 3),
        "mfma_frac": round(r["kernel_flops"] / (r["kernel_ms"] * 1e-3) / 1e12
                           / BF16_PEAK_TFLOPS, 4),
        "mfma_busy_frac_rocprof": mfma_busy_from_profiles(key),
    }


def run_workload(name, lib, pkg, rt, args, cpu_leg):
    """(metric, result, cpu_baseline) of one workload."""
    if name == "moe_decode":
        r = bench_moe_decode(lib, pkg, rt, args.steps, args.warmup)
        return ("FP8 MoE decode GEMV HBM GB/s", r,
                cpu_moe_decode(lib) if cpu_leg else None)
    if name == "moe_decode_shared":
        r = bench_moe_decode(lib, pkg, rt, args.steps, args.warmup, shared=True)
        return ("FP8 MoE decode GEMV HBM GB/s (routed + shared expert)", r,
                cpu_moe_decode(lib, shared=True) if cpu_leg else None)
    if name in ("dense_gemv", "dense_gemv_c0"):
        cfg = 0 if name == "dense_gemv_c0" else 1
        r = bench_dense_gemv(lib, pkg, rt, args.steps, args.warmup, M=args.m, cfg=cfg)
        return ("FP8 dense decode GEMV HBM GB/s", r,
                cpu_dense_gemv(lib, M=args.m, cfg=cfg) if cpu_leg else None)
    if name == "dense_gemm":
        r = bench_dense_gemm(lib, pkg, rt, args.steps, args.warmup)
        return ("FP8 dense linear GEMM TFLOP/s (DSA projections, prefill M)", r,
                cpu_dense_gemm(lib) if cpu_leg else None)
    if name == "bf16_gemv":
        r = bench_bf16_gemv(lib, pkg, rt, args.steps, args.warmup, M=args.m)
        return ("BF16 decode GEMV HBM GB/s (LM head)", r,
                cpu_bf16_gemv(lib, M=args.m) if cpu_leg else None)
    if name == "moe_decode_router":
        r = bench_moe_decode_router(lib, pkg, rt, args.steps, args.warmup)
        return ("FP8 MoE decode GEMV HBM GB/s (reference router on the GPU)", r,
                cpu_moe_decode_router(lib) if cpu_leg else None)
    if name == "store_load":
        r = bench_store_load(lib, pkg, rt, min(args.steps, 5), min(args.warmup, 1))
        return ("expert store fill GB/s (container -> HBM)", r,
                cpu_store_load(lib) if cpu_leg else None)
    if name in PREFILL:
        steps = args.prefill_steps if args.prefill_steps else args.steps
        r = bench_prefill(lib, pkg, rt, steps, min(args.warmup, PREFILL[name]["warmup"]),
                          name)
        return ("prefill grouped-GEMM TFLOP/s", r,
                cpu_moe_prefill(lib, name) if cpu_leg else None)
    r = bench_copy(rt, args.steps, args.warmup)
    return ("device copy HBM GB/s (read + write)", r, None)


def public(d):
    """d without its private (underscore) entries: the arrays a check used."""
    return None if d is None else {k: v for k, v in d.items() if not k.startswith("_")}


def line_of(metric, r, cpu, steps, warmup):
    line = {
        "metric": metric,
        "value": round(r["value"], 2),
        "unit": r.get("unit", "GB/s"),
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": r.get("data", "synthetic (include/apus_synth.h generator, seeded)"),
        "config": r["config"],
        "roofline": roofline_of(r),
        "cpu_baseline": public(cpu),
        "verified": verify(r, cpu),
    }
    if "two_launch" in r:
        line["two_launch"] = r["two_launch"]
    if "hbm_gbs" in r:
        line["hbm"] = {"achieved": round(r["hbm_gbs"], 2), "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": round(r["hbm_gbs"] / HBM_PEAK_GBS, 4),
                       "algorithmic_bytes_per_step": r["bytes"]}
    if r.get("flops") and r.get("bytes"):
        # the step against both rooflines: its time at the binding one
        # (HBM bytes at 8 TB/s or FLOPs at 2.5 PFLOP/s) over the measured time
        t_hbm = r["bytes"] / (HBM_PEAK_GBS * 1e9) * 1e3
        t_mfma = r["flops"] / (BF16_PEAK_TFLOPS * 1e12) * 1e3
        line["step_roofline"] = {
            "bound": "hbm" if t_hbm >= t_mfma else "mfma",
            "min_ms": round(max(t_hbm, t_mfma), 6),
            "frac": round(max(t_hbm, t_mfma) / r["ms_per_step"], 4),
            "hbm_frac": round(t_hbm / r["ms_per_step"], 4),
            "mfma_frac": round(t_mfma / r["ms_per_step"], 4)}
    if r.get("weight_bytes"):
        # the reference benches' accounting: weight bytes only (BF16 O*K*2,
        # tests/m3g/bench_bf16.c:122; FP8 O*K, tests/m7b/bench_gmetal.c:97-99)
        line["weight_only"] = {"bytes_per_step": r["weight_bytes"],
                               "gbs": round(r["weight_bytes"] / (r["ms_per_step"] * 1e-3)
                                            / 1e9, 2)}
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default per workload: 2000 for the "
                         "decode GEMVs, 5 for prefill, 200 otherwise)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps (default per workload: 500 for "
                         "the decode GEMVs, 2 for prefill, 20 otherwise)")
    ap.add_argument("--workload", default="moe_decode",
                    choices=["moe_decode", "moe_decode_shared", "dense_gemv", "dense_gemv_c0",
                             "dense_gemm",
                             "bf16_gemv",
                             "moe_decode_router", "store_load", "prefill_zipf",
                             "prefill_stack", "copy", "library_gemm"])
    ap.add_argument("--m", type=int, default=1,
                    help="dense_gemv / bf16_gemv rows (1, 2, 4)")
    ap.add_argument("--prefill-steps", type=int, default=0,
                    help="steps of the prefill workloads (default: --steps; "
                         "5 when they run as the metric's second half)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true",
                    help="moe_decode only: skip the prefill half of the metric")
    ap.add_argument("--no-dense", action="store_true",
                    help="moe_decode only: skip the config 0/1 dense GEMV objects")
    args = ap.parse_args()
    # The decode steps are tens of microseconds of GPU work each, launched
    # from a Python loop. The warmup runs the device into its steady state
    # before the timed steps (a store's first few thousand decode steps run
    # up to ~1.5 us slower: 500 warmup steps measured 36.2-38.0 us, 10,000
    # steps 35.7 us per decode step).
    dflt = {"moe_decode": (2000, 10000), "moe_decode_router": (2000, 10000),
            "moe_decode_shared": (2000, 10000),
            "dense_gemv": (2000, 5000), "dense_gemv_c0": (2000, 5000),
            "bf16_gemv": (2000, 500),
            "prefill_zipf": (40, 5), "prefill_stack": (5, 2),
            "library_gemm": (10, 3)}
    d_steps, d_warm = dflt.get(args.workload, (200, 20))
    if args.steps is None:
        args.steps = d_steps
    if args.warmup is None:
        args.warmup = d_warm
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(it runs on one GPU's share of the work); run --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "library_gemm":
        # torch brings its own HIP runtime: this workload runs before (and
        # without) this build's library, so only one runtime owns the device
        r = bench_library_gemm(args.steps, args.warmup)
        print(json.dumps(line_of("hipBLASLt BF16 GEMM TFLOP/s (library reference on "
                                 "the prefill shapes)", r, None, args.steps, args.warmup)))
        return
    global _LIB
    pkg, rt = load_pkg()
    lib = pkg.load()
    _LIB = lib
    err = ctypes.create_string_buffer(256)
    pkg.check(lib.apus_ghip_enable(err, 256), "apus_ghip_enable")

    metric, r, cpu = run_workload(args.workload, lib, pkg, rt, args, not args.no_cpu)
    print("bench: %s done (%.4f ms/step)" % (args.workload, r["ms_per_step"]),
          file=sys.stderr, flush=True)
    line = line_of(metric, r, cpu, args.steps, args.warmup)
    if args.workload == "moe_decode" and not args.no_dense:
        # the metric's GEMV half at the dense configs (BASELINE configs 0 and
        # 1, M = 1, 2, 4), each its own object with roofline and CPU leg.
        # Steps of a few microseconds: at least 200 timed steps each.
        line["dense"] = []
        ds, dw = max(args.steps, 200), max(args.warmup, 20)
        for cfg, M in ((0, 1), (1, 1), (1, 2), (1, 4)):
            r2 = bench_dense_gemv(lib, pkg, rt, ds, dw, M=M, cfg=cfg)
            c2 = cpu_dense_gemv(lib, M=M, cfg=cfg, budget_s=3.0) if cpu else None
            line["dense"].append(line_of("FP8 dense decode GEMV HBM GB/s", r2, c2, ds, dw))
            print("bench: config %d M=%d done (%.4f ms/step)" % (cfg, M, r2["ms_per_step"]),
                  file=sys.stderr, flush=True)
    if args.workload == "moe_decode" and not args.no_dense:
        # the decode as the model runs it: the layer's shared expert added
        # after the routed sum (c/gmoe.h:325-336), one launch
        # and routed by the reference router in the same launch
        line["decode_variants"] = []
        for name in ("moe_decode_shared", "moe_decode_router"):
            m2, r2, c2 = run_workload(name, lib, pkg, rt, args, cpu is not None)
            line["decode_variants"].append(line_of(m2, r2, c2, args.steps, args.warmup))
            print("bench: %s done (%.4f ms/step)" % (name, r2["ms_per_step"]),
                  file=sys.stderr, flush=True)
    if args.workload == "moe_decode" and not args.no_prefill:
        # the metric's second half ("...; prefill grouped-GEMM
        # TFLOP/s (%MFMA)"): configs 4 and 3, each a full step of its own
        # per config: 5 steps of config 4 (16 layers, ~60 ms each), 40 of
        # config 3 (one layer, ~2 ms each)
        fixed = args.prefill_steps
        line["prefill"] = []
        for name in ("prefill_stack", "prefill_zipf"):
            args.prefill_steps = fixed or PREFILL[name]["steps"]
            m2, r2, _ = run_workload(name, lib, pkg, rt, args, False)
            c2 = cpu_moe_prefill(lib, name) if cpu else None
            line["prefill"].append(line_of(m2, r2, c2, args.prefill_steps,
                                           min(args.warmup, PREFILL[name]["warmup"])))
            print("bench: %s done (%.4f ms/step)" % (name, r2["ms_per_step"]),
                  file=sys.stderr, flush=True)
    print(json.dumps(line))
    objs = ([line] + line.get("dense", []) + line.get("decode_variants", [])
            + line.get("prefill", []))
    bad = [o["config"].get("workload") for o in objs if not o["verified"]["ok"]]
    if bad:
        print("bench: verification failed for %s" % bad, file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
