"""The shared expert on the device (c/gmoe.h:325-336: every token runs it,
its output is added after the ascending routed combine with one more bf16
rounding and no weight), through the decode (one launch: its gate/up rows
stream while the routing runs, its down rows split over the waves) and
both prefill bodies (one more pair per token), against the oracle whose
shared-expert forward is pinned bitwise to the reference's own
apus_gmoe_forward2 (tests/test_oracle_moe.py)."""
import ctypes

import numpy as np
import pytest

import oracle as O
import gpu_util as G
from tolerance import assert_close_combined, record
from test_gpu_moe import open_store, random_slabs, status
from test_gpu_prefill import prefill

pytestmark = pytest.mark.gpu


def floor_all(slabs, shared, dim, inter, x, idx, w):
    """Floor of the combined output: each routed expert's and the shared
    expert's own floor (sum_i |h_i wd_i|) carried through the combine."""
    return O.moe_expert_floor(slabs, dim, inter, x, idx, w, threads=8, shared=shared)


def want_of(slabs, shared, dim, inter, x, idx, w):
    return O.moe_forward(slabs, dim, inter, x, idx, w, threads=8, shared=shared)


def make_store(ghip, E, dim, inter, seed, nan_shared=False):
    rng = np.random.default_rng(seed)
    slabs = random_slabs(E + 1, dim, inter, rng, nan_codes_in=(E,) if nan_shared else ())
    shared = slabs.pop()
    s = open_store(ghip, E, dim, inter)
    for e, sl in enumerate(slabs):
        assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
    assert ghip.apus_ghip_store_put_shared(s, O.ptr(shared), shared.nbytes) == 0, \
        ghip.apus_ghip_last_error()
    return s, slabs, shared, rng


@pytest.mark.parametrize("dim,inter,k,nan_shared", [(256, 128, 1, False), (256, 128, 8, True),
                                                    (256, 128, 12, False),
                                                    (4352, 128, 4, False),
                                                    (4352, 256, 11, True),
                                                    (256, 384, 8, False)])
def test_decode_shared_vs_oracle(ghip, dim, inter, k, nan_shared):
    """One token, given routing, shared expert: k = 1 and 8, more than 8
    slots (two down passes), more output row groups than workgroups, and a
    shared expert with NaN codes (its exact-decode bodies)."""
    E = 16
    s, slabs, shared, rng = make_store(ghip, E, dim, inter, dim + k, nan_shared)
    try:
        for trial in range(2):
            x = O.f32_to_bf16((rng.standard_normal(dim) * (1 + 2 * trial)).astype(np.float32))
            idx = rng.permutation(E)[:k].astype(np.int32)
            w = rng.uniform(0.05, 0.6, k).astype(np.float32)
            out = np.empty(dim, np.uint16)
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), k,
                                             O.ptr(out)) == 0, ghip.apus_ghip_last_error()
            want = want_of(slabs, shared, dim, inter, x, idx[None], w[None])
            st = assert_close_combined(out, want[0], floor_all(slabs, shared, dim, inter, x,
                                                               idx[None], w[None])[0],
                                       "decode shared dim=%d k=%d" % (dim, k))
            record("shared_decode_dim%d_inter%d_k%d_t%d" % (dim, inter, k, trial), st)
            out2 = np.empty(dim, np.uint16)
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), k,
                                             O.ptr(out2)) == 0
            assert np.array_equal(out, out2), "run-to-run determinism"
        # without the shared expert: the routed sum alone again
        assert ghip.apus_ghip_store_put_shared(s, None, 0) == 0
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), k,
                                         O.ptr(out)) == 0
        routed = O.moe_forward(slabs, dim, inter, x, idx[None], w[None], threads=8)
        assert not np.array_equal(out, want[0])
        from test_gpu_moe import moe_floor
        _, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None], threads=8,
                              want_expert_out=True)
        assert_close_combined(out, routed[0], moe_floor(eo, w[None], idx[None])[0],
                              "shared removed")
    finally:
        ghip.apus_ghip_store_close(s)


def test_decode_shared_back_to_back(ghip):
    """Shared-expert decodes enqueued back to back on one stream, the
    routed slot count changing from call to call (more than 8 slots in one
    of them): the shared expert's h words sit beside the routed slots' in
    the two alternating h buffers, and every output equals the same call
    run alone, bitwise, with no device failure recorded."""
    E, dim, inter = 16, 256, 128
    s, slabs, shared, rng = make_store(ghip, E, dim, inter, 505)
    try:
        calls = []
        for k in (8, 2, 12, 1, 8):
            x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
            idx = rng.permutation(E)[:k].astype(np.int32)
            w = rng.uniform(0.05, 0.6, k).astype(np.float32)
            calls.append((x, idx, w))
        alone = []
        for x, idx, w in calls:
            out = np.empty(dim, np.uint16)
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), len(idx),
                                             O.ptr(out)) == 0, ghip.apus_ghip_last_error()
            alone.append(out)
        bufs = [(G.dev(x), G.dev(idx), G.dev(w), G.empty(dim * 2), len(idx))
                for x, idx, w in calls]
        for dx, di, dw, do, k in bufs:
            assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), k,
                                                 G.vp(do), G.stream()) == 0
        for (dx, di, dw, do, k), want in zip(bufs, alone):
            assert np.array_equal(G.host(do, np.uint16, (dim,)), want), "k=%d" % k
        assert status(ghip, s) == 0
        x, idx, w = calls[2]
        want = want_of(slabs, shared, dim, inter, x, idx[None], w[None])
        assert_close_combined(alone[2], want[0], floor_all(slabs, shared, dim, inter, x,
                                                           idx[None], w[None])[0],
                              "shared, 12 slots")
    finally:
        ghip.apus_ghip_store_close(s)


def test_decode_shared_device_routing_and_dropped_ids(ghip):
    """Device routing from logits with the shared expert; and a call whose
    every routed id is outside the bank: the routed sum is empty (+0), the
    output is the shared expert's alone, and the status word says 2."""
    E, dim, inter, k = 16, 256, 128, 6
    s, slabs, shared, rng = make_store(ghip, E, dim, inter, 77)
    try:
        logits = rng.standard_normal(E).astype(np.float32)
        x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
        idx, w = O.route_softmax(logits, k)
        dx, dl, do = G.dev(x), G.dev(logits), G.empty(dim * 2)
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), G.vp(dl), None, None, k,
                                             G.vp(do), G.stream()) == 0
        want = want_of(slabs, shared, dim, inter, x, idx[None], w[None])
        assert_close_combined(G.host(do, np.uint16, (dim,)), want[0],
                              floor_all(slabs, shared, dim, inter, x, idx[None],
                                        w[None])[0], "shared, device routing")
        assert status(ghip, s) == 0
        bad = np.array([E, E + 1, -1], np.int32)
        wb = np.ones(3, np.float32)
        di, dw = G.dev(bad), G.dev(wb)
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), 3,
                                             G.vp(do), G.stream()) == 0
        assert status(ghip, s) == 2
        sh_only = want_of([None] * E, shared, dim, inter, x, np.full((1, 1), E + 7, np.int32),
                          np.zeros((1, 1), np.float32))
        assert_close_combined(G.host(do, np.uint16, (dim,)), sh_only[0],
                              floor_all([None] * E, shared, dim, inter, x,
                                        np.full((1, 1), E + 7, np.int32),
                                        np.zeros((1, 1), np.float32))[0],
                              "shared only")
    finally:
        ghip.apus_ghip_store_close(s)


@pytest.mark.parametrize("T,k,host", [(1, 1, True), (7, 3, False), (40, 4, True),
                                      (300, 6, False)])
def test_prefill_shared_vs_oracle(ghip, T, k, host):
    """Prefill with the shared expert: one more pair per token (the shared
    expert's rows form a tile list of their own); T = 300 at top-6 over 12
    experts takes the two-waves-per-SIMD bodies, the smaller ones the
    one-wave bodies. Repeated ids inside a token count once."""
    E, dim, inter = 12, 256, 256
    s, slabs, shared, rng = make_store(ghip, E, dim, inter, 1000 + T, nan_shared=T == 40)
    try:
        x = O.f32_to_bf16((rng.standard_normal((T, dim)) *
                           rng.uniform(0.5, 3.0, (T, 1))).astype(np.float32))
        idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
        if k > 2:
            idx[0, 1] = idx[0, 0]                      # a repeat: dropped
        w = rng.uniform(0.05, 0.6, (T, k)).astype(np.float32)
        out = prefill(ghip, s, x, idx, w, host)
        want = want_of(slabs, shared, dim, inter, x, idx, w)
        st = assert_close_combined(out, want, floor_all(slabs, shared, dim, inter, x, idx, w),
                                   "prefill shared T=%d" % T)
        record("shared_prefill_T%d_k%d" % (T, k), st)
        dec = np.empty(dim, np.uint16)
        assert ghip.apus_ghip_moe_decode(s, O.ptr(x[0]), O.ptr(idx[0]), O.ptr(w[0]), k,
                                         O.ptr(dec)) == 0
        assert_close_combined(dec, want[0], floor_all(slabs, shared, dim, inter, x[:1],
                                                      idx[:1], w[:1])[0], "decode token 0")
        assert status(ghip, s) == 0
    finally:
        ghip.apus_ghip_store_close(s)


def test_shared_real_shape(ghip, pkg):
    """BASELINE config-2 shape plus a shared expert (288 experts, dim 4096,
    inter 2048, top-8): the decode of 4 tokens and the prefill of 256 tokens
    (uniform routing: the two-waves-per-SIMD bodies) against the oracle."""
    lib = pkg.load()
    E, k, dim, inter, seed = 288, 8, 4096, 2048, 0x5C2
    s = open_store(ghip, E, dim, inter)
    try:
        assert ghip.apus_ghip_store_synth(s, seed, 0, 1e-4, 1e-2) == 0
        sb = ghip.apus_ghip_store_slab_bytes(s)
        rng = np.random.default_rng(seed)
        shared = random_slabs(1, dim, inter, rng)[0]
        assert ghip.apus_ghip_store_put_shared(s, O.ptr(shared), sb) == 0
        T = 256
        idx = np.empty((T, k), np.int32)
        w = np.empty((T, k), np.float32)
        assert lib.apus_synth_route(O.ptr(idx), O.ptr(w), T, E, k, 0.0, seed) == 0
        x = np.empty((T, dim), np.uint16)
        lib.apus_synth_bf16_normal(O.ptr(x), x.size, seed, 40, 0)
        used = sorted(set(idx.ravel().tolist()))
        slabs = [None] * E
        for e in used:
            slabs[e] = np.empty(sb, np.uint8)
            assert ghip.apus_ghip_store_get(s, e, O.ptr(slabs[e]), sb) == 0
        want = O.moe_forward(slabs, dim, inter, x, idx, w, grouped=True, threads=16,
                             shared=shared)
        fl = floor_all(slabs, shared, dim, inter, x, idx, w)
        out = prefill(ghip, s, x, idx, w, host=False)
        st = assert_close_combined(out, want, fl, "prefill shared, real shape")
        record("shared_prefill_real_shape", st)
        dec = np.empty((4, dim), np.uint16)
        for t in range(4):
            assert ghip.apus_ghip_moe_decode(s, O.ptr(x[t]), O.ptr(idx[t]), O.ptr(w[t]), k,
                                             O.ptr(dec[t])) == 0, ghip.apus_ghip_last_error()
        st = assert_close_combined(dec, want[:4], fl[:4], "decode shared, real shape")
        record("shared_decode_real_shape", st)
        assert status(ghip, s) == 0
    finally:
        ghip.apus_ghip_store_close(s)
