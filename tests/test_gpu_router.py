"""The MoE router with the reference semantics on the GPU
(apus_gmoe_router, c/gmoe.h:191-208): sigmoid scores, selection-only
bias, stable top-k (ties -> lower id), pairwise-sum normalization x 2.5,
against the oracle (pinned to the reference build in
tests/test_oracle_moe.py); then the router's output driving the MoE
decode (c/gmoe.h:294-320 after the router)."""
import ctypes

import numpy as np
import pytest

import oracle as O
import gpu_util as G
from tolerance import assert_close_combined

pytestmark = pytest.mark.gpu


def inputs(seed, E, dim, ties=False):
    rng = np.random.default_rng(seed)
    gw = O.f32_to_bf16((0.02 * rng.standard_normal((E, dim))).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    bias = (0.05 * rng.standard_normal(E)).astype(np.float32)
    if ties:
        gw[7] = gw[2]
        gw[33] = gw[2]
        bias[7] = bias[2]
        bias[33] = bias[2]
    return gw, bias, x


def gpu_router(ghip, E, topk, bias, gw=None, x=None, logits=None, scale=2.5):
    dim = gw.shape[1] if gw is not None else 0
    db = G.dev(bias)
    dgw = G.dev(gw) if gw is not None else None
    dx = G.dev(x) if x is not None else None
    dl = G.dev(logits.astype(np.float32)) if logits is not None else None
    dsc, di, dw = G.empty(E * 4), G.empty(topk * 4), G.empty(topk * 4)
    rc = ghip.apus_ghip_moe_router_dev(G.vp(dx) if dx else None, G.vp(dgw) if dgw else None,
                                       G.vp(dl) if dl else None, G.vp(db), E, dim, topk,
                                       scale, G.vp(dsc), G.vp(di), G.vp(dw), G.stream())
    assert rc == 0, ghip.apus_ghip_last_error()
    return (G.host(dsc, np.float32, (E,)), G.host(di, np.int32, (topk,)),
            G.host(dw, np.float32, (topk,)))


@pytest.mark.parametrize("E,dim,topk", [(288, 4096, 8), (64, 256, 4), (300, 512, 16),
                                        (16, 128, 1), (512, 1024, 9)])
def test_router_vs_oracle(ghip, E, dim, topk):
    gw, bias, x = inputs(E * 7 + dim + topk, E, dim)
    sc, idx, w = O.gmoe_router(gw, bias, x, topk)
    gsc, gidx, gw_ = gpu_router(ghip, E, topk, bias, gw=gw, x=x)
    # logits are a GEMV: the reference's sequential f32 sum and the GPU's
    # reordered one each sit within the f32 summation error of the exact
    # dot (|err| <~ sqrt(dim) ulps of sum_k |w x| in practice; bound here
    # 2^-16 relative to it), scores add a device expf (a few ulps);
    # sigmoid' <= 1/4
    wf = O.bf16_to_f32(gw).astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)
    absdot = np.abs(wf) @ np.abs(xf)
    tol = 0.25 * 2.0 ** -16 * absdot + 4 * 2.0 ** -24 * np.abs(sc)
    assert (np.abs(gsc.astype(np.float64) - sc) <= tol).all(), \
        np.max(np.abs(gsc.astype(np.float64) - sc) / tol)
    # the GPU scores are no further from the exact (f64) scores than the
    # reference's are, beyond the expf ulps
    ex = 1.0 / (1.0 + np.exp(-(wf @ xf)))
    slack = 4 * 2.0 ** -24 * np.abs(ex) + 1e-12
    assert (np.abs(gsc - ex) <= np.abs(sc - ex) + 0.25 * 2.0 ** -18 * absdot + slack).all()
    # no near-ties at this spacing: the same selection, in the same order
    b = np.sort(sc + bias)[::-1]
    if b[topk - 1] - b[topk] > 1e-5:
        assert np.array_equal(gidx, idx)
        assert np.allclose(gw_, w, rtol=1e-5, atol=0)


def test_router_from_logits_ties_stable(ghip):
    """Given logits (no GEMV): equal biased scores resolve to the lower id,
    and the weights are the reference's up to the device expf."""
    E, topk = 64, 6
    rng = np.random.default_rng(4)
    logits = rng.standard_normal(E).astype(np.float32)
    bias = np.zeros(E, np.float32)
    m = logits.max()
    logits[[3, 9, 40]] = m + 1.0                   # three equal leaders
    logits[[11, 12]] = m + 0.5
    sc, idx, w = O.gmoe_router_from_logits(logits, bias, topk)
    gsc, gidx, gw_ = gpu_router(ghip, E, topk, bias, logits=logits)
    assert np.array_equal(gidx, idx), (gidx, idx)
    assert list(gidx[:3]) == [3, 9, 40] and list(gidx[3:5]) == [11, 12]
    assert np.allclose(gw_, w, rtol=2e-6, atol=0)
    assert np.allclose(gsc, sc, rtol=2e-6, atol=0)


def test_router_bias_selects_not_weighs(ghip):
    E, topk = 128, 8
    rng = np.random.default_rng(8)
    logits = rng.standard_normal(E).astype(np.float32)
    bias = np.zeros(E, np.float32)
    bias[100:108] = 10.0                          # force experts 100..107
    sc, idx, w = O.gmoe_router_from_logits(logits, bias, topk)
    _, gidx, gw_ = gpu_router(ghip, E, topk, bias, logits=logits)
    assert sorted(gidx.tolist()) == list(range(100, 108))
    assert np.array_equal(gidx, idx)
    sel = sc[idx]
    assert np.allclose(gw_, sel / sel.sum() * 2.5, rtol=2e-6)


def test_router_drives_decode(ghip):
    """router -> decode on the device equals the oracle's router + expert +
    combine on the same inputs (the selection is checked exactly)."""
    E, dim, inter, topk = 16, 256, 128, 4
    rng = np.random.default_rng(21)
    slabs = []
    for e in range(E):
        parts = []
        for (o, k) in [(inter, dim), (inter, dim), (dim, inter)]:
            c = rng.integers(0, 254, (o, k), dtype=np.uint8)
            c[c >= 0x7F] += 1
            s = np.exp2(rng.uniform(-9, -5, (O.nblocks(o), O.nblocks(k)))).astype(np.float32)
            parts += [c.ravel(), s.view(np.uint8).ravel()]
        slabs.append(np.concatenate(parts))
    s = ctypes.c_void_p()
    err = ctypes.create_string_buffer(256)
    assert ghip.apus_ghip_store_open(ctypes.byref(s), E, dim, inter, 10.0, err, 256) == 0
    try:
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        gw, bias, x = inputs(5, E, dim)
        sc, idx, w = O.gmoe_router(gw, bias, x, topk)
        dgw, db, dx = G.dev(gw), G.dev(bias), G.dev(x)
        di, dw, dout = G.empty(topk * 4), G.empty(topk * 4), G.empty(dim * 2)
        assert ghip.apus_ghip_moe_router_dev(G.vp(dx), G.vp(dgw), None, G.vp(db), E, dim,
                                             topk, 2.5, None, G.vp(di), G.vp(dw),
                                             G.stream()) == 0
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), topk,
                                             G.vp(dout), G.stream()) == 0
        got = G.host(dout, np.uint16, (dim,))
        assert np.array_equal(G.host(di, np.int32, (topk,)), idx)
        want, eo = O.moe_forward(slabs, dim, inter, x, idx[None], w[None],
                                 want_expert_out=True)
        c = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo) * w[None, :, None]))
        fl = np.abs(c.astype(np.float64)).sum(1)[0]
        assert_close_combined(got, want[0], fl, "router -> decode")
    finally:
        ghip.apus_ghip_store_close(s)


def fused_case(ghip, E, dim, inter, topk, gw, bias, x, shared=None, seed=0):
    """The router-fed decode (one launch) against the two-launch form
    (router, then the decode with its picks) on the same store and inputs:
    the same picks and weights and the same outputs, bitwise; and against
    the oracle's router + experts (+ shared expert) + combine."""
    from test_gpu_moe import open_store, random_slabs
    from test_gpu_shared import floor_all
    rng = np.random.default_rng(seed)
    slabs = random_slabs(E, dim, inter, rng)
    s = open_store(ghip, E, dim, inter)
    try:
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        if shared is not None:
            assert ghip.apus_ghip_store_put_shared(s, O.ptr(shared), shared.nbytes) == 0
        dgw, db, dx = G.dev(gw), G.dev(bias), G.dev(x)
        di, dw, do1 = G.empty(topk * 4), G.empty(topk * 4), G.empty(dim * 2)
        fi, fw, do2 = G.empty(topk * 4), G.empty(topk * 4), G.empty(dim * 2)
        assert ghip.apus_ghip_moe_router_dev(G.vp(dx), G.vp(dgw), None, G.vp(db), E, dim,
                                             topk, 2.5, None, G.vp(di), G.vp(dw),
                                             G.stream()) == 0
        assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), topk,
                                             G.vp(do1), G.stream()) == 0
        assert ghip.apus_ghip_moe_decode_router_dev(s, G.vp(dx), G.vp(dgw), G.vp(db), 2.5,
                                                    topk, G.vp(do2), G.vp(fi), G.vp(fw),
                                                    G.stream()) == 0, \
            ghip.apus_ghip_last_error()
        two = (G.host(di, np.int32, (topk,)), G.host(dw, np.float32, (topk,)),
               G.host(do1, np.uint16, (dim,)))
        one = (G.host(fi, np.int32, (topk,)), G.host(fw, np.float32, (topk,)),
               G.host(do2, np.uint16, (dim,)))
        for a, b, what in zip(two, one, ("idx", "w", "out")):
            assert np.array_equal(a, b), "fused vs two launches: " + what
        code = ctypes.c_uint32(1)
        assert ghip.apus_ghip_store_status(s, None, 1, ctypes.byref(code)) == 0
        assert code.value == 0
        sc, idx, w = O.gmoe_router(gw, bias, x, topk)
        want = O.moe_forward(slabs, dim, inter, x, idx[None], w[None], threads=8,
                             shared=shared)
        fl = floor_all(slabs, shared, dim, inter, x, idx[None], w[None])[0]
        return one, idx, w, want[0], fl
    finally:
        ghip.apus_ghip_store_close(s)


@pytest.mark.parametrize("E,dim,inter,topk", [(288, 4096, 256, 8), (64, 256, 128, 4),
                                              (300, 512, 128, 16), (16, 128, 128, 1),
                                              (512, 1024, 128, 9)])
def test_router_fused_decode(ghip, E, dim, inter, topk):
    gw, bias, x = inputs(E * 5 + dim + topk, E, dim)
    (gidx, gwt, out), idx, w, want, fl = fused_case(ghip, E, dim, inter, topk, gw, bias, x,
                                                    seed=E + topk)
    b = np.sort(O.gmoe_router(gw, bias, x, topk)[0] + bias)[::-1]
    if b[topk - 1] - b[topk] > 1e-5:                 # no near-tie at this spacing
        assert np.array_equal(gidx, idx)
        assert np.allclose(gwt, w, rtol=1e-5, atol=0)
        assert_close_combined(out, want, fl, "fused router decode E=%d" % E)


def test_router_fused_ties_and_bias(ghip):
    """Through the one-launch path: equal gate rows (equal logits and biases)
    resolve to the lower id, in the reference's order; a bias that selects
    experts 100..107 selects them but does not weigh them."""
    E, dim, inter, topk = 128, 256, 128, 6
    gw, bias, x = inputs(31, E, dim, ties=True)
    gw[[2, 7, 33]] = O.f32_to_bf16(np.full(dim, 0.5, np.float32) * np.sign(
        O.bf16_to_f32(x)))                            # the three tied rows lead
    (gidx, gwt, out), idx, w, want, fl = fused_case(ghip, E, dim, inter, topk, gw, bias, x)
    assert list(gidx[:3]) == [2, 7, 33]
    assert np.array_equal(gidx, idx)
    assert np.allclose(gwt, w, rtol=1e-5, atol=0)
    assert_close_combined(out, want, fl, "ties")
    gw, bias, x = inputs(32, E, dim)
    bias[:] = 0.0
    bias[100:108] = 10.0
    (gidx, gwt, out), idx, w, want, fl = fused_case(ghip, E, dim, inter, 8, gw, bias, x)
    assert sorted(gidx.tolist()) == list(range(100, 108))
    sc = O.gmoe_router(gw, bias, x, 8)[0]
    assert np.allclose(gwt, sc[gidx] / sc[gidx].sum() * 2.5, rtol=2e-6)
    assert_close_combined(out, want, fl, "bias selects")


def test_router_fused_decode_with_shared_expert(ghip):
    """The whole MoE sublayer of c/gmoe.h:265-337 in one launch: router,
    routed experts, shared expert."""
    from test_gpu_moe import random_slabs
    E, dim, inter, topk = 64, 512, 256, 8
    gw, bias, x = inputs(77, E, dim)
    shared = random_slabs(1, dim, inter, np.random.default_rng(78))[0]
    (gidx, gwt, out), idx, w, want, fl = fused_case(ghip, E, dim, inter, topk, gw, bias, x,
                                                    shared=shared, seed=79)
    assert np.array_equal(gidx, idx)
    assert_close_combined(out, want, fl, "router + routed + shared, one launch")
