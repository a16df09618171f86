"""Pins of the oracle's SwiGLU expert, combine and routing — CPU only.

sigmoid: c/gmhc.h:157-160 (and the reference build). pw_sum: numpy's own
float32 pairwise sum, which c/gmhc.h:165-185 replicates. top-k: a stable
argsort (descending value, ties -> lower index), c/gmoe.h:175-189. expert:
golden fixtures written by the reference's apus_gmoe_expert
(c/gmoe.h:210-227). combine: order/rounding invariants of c/gmoe.h:307-320
and the config-2 golden (reference expert outputs, reference loop).
"""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def fx():
    return np.load(os.path.join(GOLD, "fixtures.npz"))


@pytest.fixture(scope="module")
def man():
    with open(os.path.join(GOLD, "manifest.json")) as f:
        return json.load(f)


def test_sigmoid_closed_form():
    L = O.lib()
    for x in [-30.0, -10.0, -1.5, -1e-3, 0.0, 1e-3, 0.75, 10.0, 30.0]:
        want = 1.0 / (1.0 + np.exp(-x))
        assert abs(L.apo_sigmoid_np(x) - want) <= 2e-7 * max(1.0, want)
    if O.ref_available():
        R = O.ref()
        for x in np.linspace(-20, 20, 4001, dtype=np.float32):
            assert L.apo_sigmoid_np(float(x)) == R.ref_sigmoid(float(x))


@pytest.mark.parametrize("n", [1, 2, 7, 8, 9, 16, 31, 128, 129, 300, 1000])
def test_pw_sum_is_numpy_pairwise(n):
    a = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    got = O.lib().apo_pw_sum(O.ptr(a), n)
    assert np.float32(got) == np.add.reduce(a, dtype=np.float32)


def test_topk_stable():
    rng = np.random.default_rng(5)
    L = O.lib()
    for trial in range(50):
        n = int(rng.integers(8, 300))
        row = rng.integers(-5, 5, n).astype(np.float32)   # many ties
        k = int(rng.integers(1, 9))
        idx = np.empty(k, np.int32)
        L.apo_topk_stable(O.ptr(row), n, k, O.ptr(idx))
        want = np.argsort(-row, kind="stable")[:k]
        assert np.array_equal(idx, want)
        if O.ref_available():
            ridx = np.empty(k, np.int32)
            O.ref().ref_topk_stable(O.ptr(row), n, k, O.ptr(ridx))
            assert np.array_equal(idx, ridx)


def test_route_softmax():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal(288).astype(np.float32)
    idx, w = O.route_softmax(logits, 8)
    assert np.array_equal(idx, np.argsort(-logits, kind="stable")[:8])
    sel = logits[idx].astype(np.float64)
    want = np.exp(sel - sel.max()) / np.exp(sel - sel.max()).sum()
    assert np.allclose(w, want, rtol=1e-6, atol=0)
    assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6


def _router_inputs(seed, E, dim, ties=False):
    rng = np.random.default_rng(seed)
    gw = O.f32_to_bf16((0.02 * rng.standard_normal((E, dim))).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    if ties:
        # equal gate rows and equal biases: equal biased scores, so the stable
        # order (lower id first) decides
        gw[5] = gw[3]
        gw[40] = gw[3]
        bias = np.zeros(E, np.float32)
    else:
        bias = (0.05 * rng.standard_normal(E)).astype(np.float32)
    return gw, bias, x


@pytest.mark.parametrize("E,dim,topk,ties", [(288, 4096, 8, False), (64, 256, 4, True),
                                             (288, 512, 8, True), (16, 128, 1, False),
                                             (300, 256, 16, False)])
def test_router_closed_form(E, dim, topk, ties):
    """The oracle router against a float64/numpy restatement: sequential
    fp32 dots equal np.cumsum order, sigmoid, selection on score + bias
    (stable argsort), weights = selected scores / (pairwise sum + 1e-20) *
    2.5; and against the reference build bitwise."""
    gw, bias, x = _router_inputs(E * 31 + dim, E, dim, ties)
    sc, idx, w = O.gmoe_router(gw, bias, x, topk)
    # sequential fp32 dot: numpy's cumulative float32 sum is the same order
    prod = (O.bf16_to_f32(gw) * O.bf16_to_f32(x)[None, :]).astype(np.float32)
    logits = np.cumsum(prod, axis=1, dtype=np.float32)[:, -1]
    want_sc = np.array([O.lib().apo_sigmoid_np(float(v)) for v in logits], np.float32)
    assert np.array_equal(sc, want_sc)
    b = (want_sc + bias).astype(np.float32)
    assert np.array_equal(idx, np.argsort(-b, kind="stable")[:topk])
    sel = want_sc[idx]
    den = np.float32(np.add.reduce(sel, dtype=np.float32) + np.float32(1e-20))
    assert np.array_equal(w, (sel / den * np.float32(2.5)).astype(np.float32))
    if ties:
        assert list(idx).index(3) < list(idx).index(5) if 5 in idx and 3 in idx else True
    if O.ref_available():
        rsc = np.empty(E, np.float32)
        ridx = np.empty(topk, np.int32)
        rw = np.empty(topk, np.float32)
        O.ref().ref_gmoe_router(O.ptr(gw), O.ptr(bias), E, dim, topk, 2.5, O.ptr(x),
                                O.ptr(rsc), O.ptr(ridx), O.ptr(rw))
        assert np.array_equal(sc, rsc) and np.array_equal(idx, ridx)
        assert np.array_equal(w, rw)
    # from logits: the same selection and weights
    sc2, idx2, w2 = O.gmoe_router_from_logits(logits, bias, topk)
    assert np.array_equal(idx2, idx) and np.array_equal(w2, w) and np.array_equal(sc2, sc)


def test_router_planted_bias_mistake_is_detected():
    """The bias selects but never weighs: a router that weighs by the
    biased score would differ (the check above pins this)."""
    gw, bias, x = _router_inputs(77, 288, 512)
    bias = bias + np.float32(0.5)
    sc, idx, w = O.gmoe_router(gw, bias, x, 8)
    bad = (sc[idx] + bias[idx]) / np.float32((sc[idx] + bias[idx]).sum() + 1e-20) * 2.5
    assert not np.allclose(w, bad, rtol=1e-3)


def test_expert_golden(fx, man):
    for i, sh in enumerate(man["expert"]):
        pl = [O.dequant(fx[f"xp{i}_{nm}_codes"], fx[f"xp{i}_{nm}_scales"])
              for nm in "gud"]
        out, g, u, h = O.swiglu_expert(pl[0], pl[1], pl[2], fx[f"xp{i}_x"])
        assert np.array_equal(out, fx[f"xp{i}_out"]), sh
        out_mt = O.swiglu_expert(pl[0], pl[1], pl[2], fx[f"xp{i}_x"], threads=4)[0]
        assert np.array_equal(out_mt, out), sh
        if sh["x_std"] > 4:
            gf, uf = O.bf16_to_f32(g), O.bf16_to_f32(u)
            assert (gf > 10).any() and (np.abs(uf) > 10).any(), "clamps must fire"


def _bank(dim, inter, E, rng):
    from test_oracle_dequant_gemm import deq_exact_f64  # noqa: F401
    slabs = []
    for e in range(E):
        parts = []
        for (o, k) in [(inter, dim), (inter, dim), (dim, inter)]:
            c = rng.integers(0, 254, (o, k), dtype=np.uint8)
            c[c >= 0x7F] += 1
            s = np.exp2(rng.uniform(-9, -5, (O.nblocks(o), O.nblocks(k)))).astype(np.float32)
            parts += [c.ravel(), s.view(np.uint8).ravel()]
        slabs.append(np.concatenate(parts))
    return slabs


def _expert_of(slab, dim, inter):
    n = inter * dim
    nbs = O.nblocks(inter) * O.nblocks(dim) * 4
    gw = slab[:n].reshape(inter, dim)
    gs = slab[n:n + nbs].view(np.float32).reshape(O.nblocks(inter), O.nblocks(dim))
    uw = slab[n + nbs:2 * n + nbs].reshape(inter, dim)
    us = slab[2 * n + nbs:2 * n + 2 * nbs].view(np.float32).reshape(gs.shape)
    dw = slab[2 * n + 2 * nbs:3 * n + 2 * nbs].reshape(dim, inter)
    ds = slab[3 * n + 2 * nbs:].view(np.float32).reshape(O.nblocks(dim), O.nblocks(inter))
    return O.dequant(gw, gs), O.dequant(uw, us), O.dequant(dw, ds)


def test_moe_combine_semantics():
    """Combine = ascending expert id, contrib = bf16(out_e * w), y = bf16(y +
    contrib): checked by recomputing from per-expert outputs, slot-order
    invariance, and k = 1 reducing to bf16(out * w)."""
    dim, inter, E, k = 128, 64, 12, 6
    rng = np.random.default_rng(21)
    slabs = _bank(dim, inter, E, rng)
    T = 5
    x = O.f32_to_bf16(rng.standard_normal((T, dim)).astype(np.float32) * 3)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.05, 0.6, (T, k)).astype(np.float32)
    out, eo = O.moe_forward(slabs, dim, inter, x, idx, w, want_expert_out=True)
    for t in range(T):
        y = np.zeros(dim, np.float32)
        for j in np.argsort(idx[t]):
            pg, pu, pd = _expert_of(slabs[idx[t, j]], dim, inter)
            assert np.array_equal(O.swiglu_expert(pg, pu, pd, x[t])[0], eo[t, j])
            c = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo[t, j]) * w[t, j]))
            y = O.bf16_to_f32(O.f32_to_bf16(y + c))
        assert np.array_equal(O.f32_to_bf16(y), out[t])
    perm = rng.permutation(k)
    out2 = O.moe_forward(slabs, dim, inter, x, idx[:, perm].copy(),
                         w[:, perm].copy())
    assert np.array_equal(out, out2)
    out1, eo1 = O.moe_forward(slabs, dim, inter, x, idx[:, :1].copy(),
                              w[:, :1].copy(), want_expert_out=True)
    assert np.array_equal(out1, O.f32_to_bf16(O.bf16_to_f32(eo1[:, 0]) * w[:, :1]))


def test_moe_planted_order_mistake_is_detected():
    """Descending-order combine differs from ascending on some token: the
    order pin bites (bf16 rounding per add is not associative)."""
    dim, inter, E, k = 128, 64, 10, 8
    rng = np.random.default_rng(4)
    slabs = _bank(dim, inter, E, rng)
    x = O.f32_to_bf16(rng.standard_normal((4, dim)).astype(np.float32) * 4)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(4)]).astype(np.int32)
    w = rng.uniform(0.05, 0.6, (4, k)).astype(np.float32)
    out, eo = O.moe_forward(slabs, dim, inter, x, idx, w, want_expert_out=True)
    differs = False
    for t in range(4):
        y = np.zeros(dim, np.float32)
        for j in np.argsort(idx[t])[::-1]:
            c = O.bf16_to_f32(O.f32_to_bf16(O.bf16_to_f32(eo[t, j]) * w[t, j]))
            y = O.bf16_to_f32(O.f32_to_bf16(y + c))
        differs |= not np.array_equal(O.f32_to_bf16(y), out[t])
    assert differs


@pytest.mark.skipif(not O.ref_available(), reason="reference build absent")
def test_expert_vs_reference_build_real_shape():
    R = O.ref()
    rng = np.random.default_rng(17)
    dim, inter = 4096, 2048
    pl = [O.f32_to_bf16((rng.standard_normal((o, k)) * 0.02).astype(np.float32))
          for (o, k) in [(inter, dim), (inter, dim), (dim, inter)]]
    x = O.f32_to_bf16(rng.standard_normal(dim).astype(np.float32))
    out_ref = np.empty(dim, np.uint16)
    assert R.ref_gmoe_expert(O.ptr(pl[0]), O.ptr(pl[1]), O.ptr(pl[2]), O.ptr(x),
                             dim, inter, 10.0, O.ptr(out_ref)) == 0
    assert np.array_equal(O.swiglu_expert(*pl, x, threads=8)[0], out_ref)


def test_slab_layout_arithmetic():
    """Slab = gate.w | gate.s | up.w | up.s | down.w | down.s
    (c/gcache.h:852-861); 25,171,968 B at dim 4096 / inter 2048
    (tests/m1/README.md:77-78 of the reference); ragged scale grids use
    ceil(n/128)."""
    L = O.lib().apo_slab_layout(4096, 2048)
    assert L.bytes == 25_171_968
    assert (L.gw, L.gs, L.uw) == (0, 8_388_608, 8_388_608 + 2048)
    assert L.us == L.uw + 8_388_608 and L.dw == L.us + 2048
    assert L.ds == L.dw + 8_388_608 and L.bytes == L.ds + 2048
    r = O.lib().apo_slab_layout(200, 136)       # inter 136 -> 2 blocks, dim 2
    nb = 2 * 2 * 4
    assert r.bytes == 2 * (136 * 200 + nb) + 200 * 136 + nb


@pytest.mark.parametrize("dim,inter", [(256, 128), (130, 70)])
def test_grouped_forward_equals_per_token_loop(dim, inter):
    """apo_moe_forward_grouped (expert by expert, M-row GEMMs) returns the
    per-token loop's bits: outputs and per-pair expert outputs, with
    repeated ids (first slot kept), ids outside the bank (dropped), ragged
    experts (some empty, one in every token), ragged shapes (row counts and
    output widths off the 8-row and 4-column blocks) and a thread-count
    change."""
    E, k, T = 9, 4, 37
    rng = np.random.default_rng(99)
    slabs = _bank(dim, inter, E, rng)
    x = O.f32_to_bf16((rng.standard_normal((T, dim)) * 2).astype(np.float32))
    idx = np.stack([np.concatenate([[2], rng.permutation([e for e in range(E - 2)
                                                          if e != 2])[:k - 1]])
                    for _ in range(T)]).astype(np.int32)
    idx[3] = [5, 5, 1, 5]                               # repeats
    idx[7, 2] = E + 3                                   # outside the bank
    w = rng.uniform(0.05, 0.6, (T, k)).astype(np.float32)
    want, eo = O.moe_forward(slabs, dim, inter, x, idx, w, want_expert_out=True)
    for th in (1, 5):
        got, geo = O.moe_forward(slabs, dim, inter, x, idx, w, want_expert_out=True,
                                 grouped=True, threads=th)
        assert np.array_equal(got, want)
        for t in range(T):
            seen = set()
            for j in range(k):
                e = int(idx[t, j])
                if 0 <= e < E and e not in seen:
                    assert np.array_equal(geo[t, j], eo[t, j]), (t, j)
                seen.add(e)


def test_chain64_yardstick_matches_numpy_f64():
    """The f64-sum yardstick (apo_moe_chain64_grouped) against the same chain
    written with numpy's f64 matmuls: one expert, top-1, weight 1, so the
    output is the expert's own. The sums differ only in f64 order, far
    below the f32 rounding that follows: equal almost everywhere, never
    more than one bf16 ulp apart; and it is a different yardstick from the
    fp32 oracle (some outputs differ)."""
    dim, inter, T = 512, 256, 24
    rng = np.random.default_rng(64)
    slabs = _bank(dim, inter, 1, rng)
    x = O.f32_to_bf16((rng.standard_normal((T, dim)) * 3).astype(np.float32))
    idx = np.zeros((T, 1), np.int32)
    w = np.ones((T, 1), np.float32)
    got = O.moe_forward(slabs, dim, inter, x, idx, w, chain64=True, threads=4)
    pl = np.empty(3 * inter * dim, np.uint16)
    O.lib().apo_slab_dequant(O.ptr(slabs[0]), dim, inter, O.ptr(pl), 1)
    f = O.bf16_to_f32(pl).astype(np.float64)
    wg, wu = f[:inter * dim].reshape(inter, dim), f[inter * dim:2 * inter * dim].reshape(inter, dim)
    wd = f[2 * inter * dim:].reshape(dim, inter)
    r = lambda v: O.bf16_to_f32(O.f32_to_bf16(np.asarray(v, np.float32)))  # noqa: E731
    xf = O.bf16_to_f32(x).astype(np.float64)
    g = np.minimum(r(xf @ wg.T), np.float32(10))
    u = np.clip(r(xf @ wu.T), -10, 10).astype(np.float32)
    sig = np.vectorize(lambda v: O.lib().apo_sigmoid_np(float(v)), otypes=[np.float32])
    h = r(r(g * sig(g)) * u)
    want = O.f32_to_bf16((h.astype(np.float64) @ wd.T).astype(np.float32))
    from tolerance import bf16_ord
    d = np.abs(bf16_ord(got) - bf16_ord(want))
    assert d.max() <= 1 and (d == 0).mean() >= 0.999, (d.max(), (d == 0).mean())
    f32 = O.moe_forward(slabs, dim, inter, x, idx, w, grouped=True, threads=4)
    assert not np.array_equal(f32, got)


def test_expert_floor_helper():
    """moe_expert_floor = sum over a token's kept pairs of |w_e| * sum_i
    |h_i * wd_e[j, i]|, recomputed from the oracle's own h (swiglu_expert)
    and the dequantized down weights in numpy (the helper rounds each
    expert's sum to bf16: within 2^-8 relative)."""
    dim, inter, E, k, T = 128, 64, 6, 3, 5
    rng = np.random.default_rng(7)
    slabs = _bank(dim, inter, E, rng)
    x = O.f32_to_bf16((rng.standard_normal((T, dim)) * 2).astype(np.float32))
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    idx[1, 2] = idx[1, 0]                               # a repeat counts once
    w = rng.uniform(-0.6, 0.6, (T, k)).astype(np.float32)
    got = O.moe_expert_floor(slabs, dim, inter, x, idx, w, threads=2)
    want = np.zeros((T, dim))
    for t in range(T):
        seen = set()
        for j in range(k):
            e = int(idx[t, j])
            if e in seen:
                continue
            seen.add(e)
            pg, pu, pd = _expert_of(slabs[e], dim, inter)
            h = O.swiglu_expert(pg, pu, pd, x[t])[3]
            F = np.abs(O.bf16_to_f32(pd).astype(np.float64)) @ np.abs(
                O.bf16_to_f32(h).astype(np.float64))
            want[t] += abs(float(w[t, j])) * F
    assert np.allclose(got, want, rtol=2.0 ** -8, atol=0)


def _payload_of(slab, dim, inter):
    pl = np.empty(3 * inter * dim, np.uint16)
    O.lib().apo_slab_dequant(O.ptr(slab), dim, inter, O.ptr(pl), 1)
    return pl


@pytest.mark.skipif(not O.ref_available(), reason="reference build absent")
def test_shared_expert_forward_vs_reference_forward2():
    """The whole MoE sublayer of the reference (apus_gmoe_forward2,
    c/gmoe.h:265-337: router, routed experts in ascending id, the shared
    expert added last with one more bf16 rounding), built from the
    reference sources, against the oracle's router (apo_gmoe_router) feeding
    apo_moe_forward_shared, and the grouped form: bitwise, on payloads
    dequantized from FP8 slabs (c/gmodel.h:962-997 dequantizes the shared
    expert at open)."""
    dim, inter, E, k, T = 256, 128, 12, 4, 9
    rng = np.random.default_rng(325)
    slabs = _bank(dim, inter, E, rng)
    shared = _bank(dim, inter, 1, rng)[0]
    gate_w = O.f32_to_bf16((rng.standard_normal((E, dim)) / 16).astype(np.float32))
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    x = O.f32_to_bf16((rng.standard_normal((T, dim)) * 2).astype(np.float32))
    pls = [_payload_of(s, dim, inter) for s in slabs]
    spl = _payload_of(shared, dim, inter)
    arr = (ctypes.c_void_p * E)(*[p.ctypes.data for p in pls])
    ref = np.empty((T, dim), np.uint16)
    ridx = np.empty((T, k), np.int32)
    rw = np.empty((T, k), np.float32)
    O.ref().ref_gmoe_forward2(arr, E, dim, inter, O.ptr(spl), inter, 10.0, O.ptr(gate_w),
                              O.ptr(bias), k, 2.5, O.ptr(x), T, O.ptr(ref), O.ptr(ridx),
                              O.ptr(rw))
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    for t in range(T):
        _, idx[t], w[t] = O.gmoe_router(gate_w, bias, x[t], k, 2.5)
    assert np.array_equal(idx, ridx) and np.array_equal(w, rw)
    got = O.moe_forward(slabs, dim, inter, x, idx, w, shared=shared)
    assert np.array_equal(got, ref)
    grp = O.moe_forward(slabs, dim, inter, x, idx, w, shared=shared, grouped=True, threads=3)
    assert np.array_equal(grp, ref)
    # the shared add is a real step: without it the outputs differ
    assert not np.array_equal(O.moe_forward(slabs, dim, inter, x, idx, w), ref)
