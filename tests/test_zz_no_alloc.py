"""The allocation-free prefill entry point (apus_ghip_moe_prefill_dev_noalloc)
against the existing apus_ghip_moe_prefill_dev on the same inputs: bitwise
equal outputs on two calls in a row (the second smaller, so the fixed
workspace holds the first call's leftovers), the device's free memory
unchanged across the no-alloc calls (they allocate nothing, whatever the
regular workspace holds), one call past the fixed workspace rejected with a
clear error, and a prefill through the regular entry point in between that
leaves the no-alloc workspace to itself."""
import ctypes

import numpy as np
import pytest

import oracle as O
import gpu_util as G
from tolerance import assert_close_combined
from test_gpu_moe import open_store, random_slabs
from test_gpu_prefill import floor_of, skewed_routing

pytestmark = pytest.mark.gpu


def run(ghip, fn, s, x, idx, w):
    T, k = idx.shape
    dim = x.shape[1]
    dx, di, dw, do = G.dev(x), G.dev(idx), G.dev(w), G.empty(T * dim * 2)
    rc = fn(s, G.vp(dx), T, G.vp(di), G.vp(dw), k, G.vp(do), G.stream())
    assert rc == 0, ghip.apus_ghip_last_error()
    return G.host(do, np.uint16, (T, dim))


def test_noalloc_prefill_matches_regular(ghip):
    E, dim, inter = 12, 256, 256
    rng = np.random.default_rng(0x0A)
    slabs = random_slabs(E, dim, inter, rng, nan_codes_in=(4,))
    s = open_store(ghip, E, dim, inter)
    try:
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        cases = []
        for T, k, hot in ((300, 6, 4), (37, 3, 1)):          # second call smaller
            x = O.f32_to_bf16(rng.standard_normal((T, dim)).astype(np.float32))
            idx, w = skewed_routing(rng, T, E, k, hot=hot)
            cases.append((x, idx, w))
        # the no-alloc calls come first in the process's life of this store
        # and allocate nothing: the device's free memory is the same before
        # and after them (their buffers are allocated beforehand)
        bufs = [(G.dev(x), G.dev(idx), G.dev(w), G.empty(idx.shape[0] * dim * 2), idx.shape)
                for x, idx, w in cases]
        G.rt().synchronize()
        free0 = G.rt().mem_info()[0]
        for dx, di, dw, do, (T, k) in bufs:
            rc = ghip.apus_ghip_moe_prefill_dev_noalloc(s, G.vp(dx), T, G.vp(di), G.vp(dw),
                                                        k, G.vp(do), G.stream())
            assert rc == 0, ghip.apus_ghip_last_error()
        G.rt().synchronize()
        assert G.rt().mem_info()[0] == free0, "the no-alloc entry point allocated"
        got = [G.host(do, np.uint16, (T, dim)) for _, _, _, do, (T, k) in bufs]
        ref = [run(ghip, ghip.apus_ghip_moe_prefill_dev, s, *c) for c in cases]
        for (x, idx, w), g, r in zip(cases, got, ref):
            assert np.array_equal(g, r), "T=%d: no-alloc differs from the regular entry" % len(x)
        # and against the oracle (the tolerance of every prefill test)
        x, idx, w = cases[1]
        want, eo = O.moe_forward(slabs, dim, inter, x, idx, w, want_expert_out=True)
        assert_close_combined(got[1], want, floor_of(eo, w, idx), "no-alloc vs oracle")
        # repeat the first (larger) call after the smaller one: same bits
        assert np.array_equal(run(ghip, ghip.apus_ghip_moe_prefill_dev_noalloc, s,
                                  *cases[0]), ref[0])
    finally:
        ghip.apus_ghip_store_close(s)


def test_noalloc_prefill_rejects_oversize(ghip):
    """A call whose workspace exceeds the fixed array is refused before any
    launch, with the needed size in the error."""
    E, dim, inter = 8, 4096, 2048
    s = open_store(ghip, E, dim, inter)
    try:
        T, k = 4096, 8                                 # 32768 pairs: ~400 MB
        x = np.zeros((T, dim), np.uint16)
        idx = np.tile(np.arange(k, dtype=np.int32), (T, 1))
        w = np.full((T, k), 0.125, np.float32)
        dx, di, dw, do = G.dev(x), G.dev(idx), G.dev(w), G.empty(T * dim * 2)
        rc = ghip.apus_ghip_moe_prefill_dev_noalloc(s, G.vp(dx), T, G.vp(di), G.vp(dw), k,
                                                    G.vp(do), G.stream())
        assert rc != 0
        assert b"fixed" in ghip.apus_ghip_last_error()
    finally:
        ghip.apus_ghip_store_close(s)


def test_noalloc_prefill_graph_replay(ghip):
    """The allocation-free entry point inside a HIP graph: two calls (a
    sparse and a full-tile routing) captured on a stream, the graph replayed
    four times with eager calls on the same fixed workspace in between, and
    every replay's outputs equal to the eager ones, bitwise (the per-call
    state -- header, queue counters, tile list -- is rebuilt by kernels in
    the graph, with no memset nodes)."""
    E, dim, inter = 12, 256, 256
    rt = G.rt()
    rng = np.random.default_rng(0x6A)
    slabs = random_slabs(E, dim, inter, rng, nan_codes_in=(4,))
    s = open_store(ghip, E, dim, inter)
    g = None
    try:
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        cases = []
        for T, k, hot in ((40, 4, 2), (300, 6, 4)):        # sparse, then full tiles
            x = O.f32_to_bf16(rng.standard_normal((T, dim)).astype(np.float32))
            idx, w = skewed_routing(rng, T, E, k, hot=hot)
            cases.append((x, idx, w))
        want = [run(ghip, ghip.apus_ghip_moe_prefill_dev_noalloc, s, *c) for c in cases]
        bufs = [(G.dev(x), G.dev(idx), G.dev(w), G.empty(len(x) * dim * 2), idx.shape)
                for x, idx, w in cases]
        st = rt.Stream()
        g = rt.Graph(st)
        g.begin()
        rcs = []
        try:
            for dx, di, dw, do, (T, k) in bufs:
                rcs.append(ghip.apus_ghip_moe_prefill_dev_noalloc(
                    s, G.vp(dx), T, G.vp(di), G.vp(dw), k, G.vp(do), st.vp))
        finally:
            g.end()
        assert rcs == [0, 0], ghip.apus_ghip_last_error()
        for rep in range(4):
            for *_, do, _ in bufs:
                do.zero()
            g.launch()
            st.synchronize()
            for n, ((_, _, _, do, (T, k)), ref) in enumerate(zip(bufs, want)):
                assert np.array_equal(G.host(do, np.uint16, (T, dim)), ref), \
                    "replay %d, call %d (T=%d)" % (rep, n, T)
            c = cases[rep % 2]                           # eager work between replays
            assert np.array_equal(run(ghip, ghip.apus_ghip_moe_prefill_dev_noalloc, s, *c),
                                  want[rep % 2])
    finally:
        if g is not None:
            g.close()
        ghip.apus_ghip_store_close(s)
