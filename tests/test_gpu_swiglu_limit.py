"""The SwiGLU clamps (c/gmoe.h:217-222: gate clamped above, up clamped on
both sides, before the silu) at limits tight enough that most g and u
values clamp, through the decode launch (K3) and both prefill tile bodies
(K4: 4-wave bodies for a ragged routing, 8-wave bodies for full tiles),
against the oracle's per-token loop at the same limit. Each case also
checks, with the oracle's own g and u, that the clamps fire on both
sides, and that the output differs from the one at the default limit, so
the store's limit is the one the kernels use.

Floor: at such limits every h_i sits near +-limit * silu(limit), and each
expert's down GEMM cancels deeply (an output of -0.39 from terms whose
|sum| is 19.8), so a one-ulp step of one h_i -- a legitimate difference of
the GPU's own gate/up GEMM -- moves the combined output by up to
w_e * 2^-8 * sum_i |h_i * wd_i|, which the combine's floor sum_e |contrib_e|
does not see. The floor here is therefore sum_e w_e * sum_i |h_i * wd_i|
(the expert-output floor of tests/tolerance.py, carried through the
combine) where that is larger. A wrong clamp moves h_i by O(limit) on
about half the elements and the outputs by O(floor)."""
import numpy as np
import pytest

import oracle as O
from test_gpu_moe import open_store, random_slabs, moe_floor
from test_gpu_prefill import prefill, floor_of, skewed_routing
from tolerance import assert_close_combined, record

pytestmark = pytest.mark.gpu

E, DIM, INTER = 6, 256, 256


def split_slab(sl):
    """(wg, wu, wd) dequantized to bf16 from one expert slab."""
    out, off = [], 0
    for (o, k) in [(INTER, DIM), (INTER, DIM), (DIM, INTER)]:
        c = sl[off:off + o * k].reshape(o, k)
        off += o * k
        ns = O.nblocks(o) * O.nblocks(k)
        s = sl[off:off + 4 * ns].view(np.float32).reshape(O.nblocks(o), O.nblocks(k))
        off += 4 * ns
        out.append(O.dequant(c, s))
    return out


@pytest.fixture(scope="module")
def slabs():
    return random_slabs(E, DIM, INTER, np.random.default_rng(91))


@pytest.fixture(scope="module", params=[0.5, 4.0])
def store(ghip, slabs, request):
    limit = request.param
    stores = {}
    for lim in (limit, 10.0):
        s = open_store(ghip, E, DIM, INTER, limit=lim)
        for e, sl in enumerate(slabs):
            assert ghip.apus_ghip_store_put(s, e, O.ptr(sl), sl.nbytes) == 0
        stores[lim] = s
    yield ghip, stores, limit
    for s in stores.values():
        ghip.apus_ghip_store_close(s)


def oracle_inner(slabs, x, idx, w, limit):
    """(floor [T, DIM] = sum_j w_tj * sum_i |h_i * wd_ci| over the token's
    experts, and the fractions of their g above limit, u above limit and u
    below -limit), from the oracle's g, u and h (before the clamps for g
    and u)."""
    W = [split_slab(sl) for sl in slabs]
    T, k = idx.shape
    floor = np.zeros((T, DIM))
    gs, us = [], []
    for t in range(T):
        for j in range(k):
            wg, wu, wd = W[idx[t, j]]
            _, g, u, h = O.swiglu_expert(wg, wu, wd, x[t], limit)
            gs.append(O.bf16_to_f32(g))
            us.append(O.bf16_to_f32(u))
            hd = np.abs(O.bf16_to_f32(h).astype(np.float64))
            floor[t] += w[t, j] * (np.abs(O.bf16_to_f32(wd).astype(np.float64)) @ hd)
    g, u = np.concatenate(gs), np.concatenate(us)
    return floor, ((g > limit).mean(), (u > limit).mean(), (u < -limit).mean())


def test_decode_clamps(store, slabs):
    ghip, stores, limit = store
    rng = np.random.default_rng(int(limit * 8))
    for trial in range(3):
        x = O.f32_to_bf16(rng.standard_normal(DIM).astype(np.float32))
        idx = rng.permutation(E)[:4].astype(np.int32)
        w = rng.uniform(0.05, 1.0, 4).astype(np.float32)
        inner, frac = oracle_inner(slabs, x[None], idx[None], w[None], limit)
        assert min(frac) > 0.05, frac
        outs = {}
        for lim, s in stores.items():
            out = np.empty(DIM, np.uint16)
            rc = ghip.apus_ghip_moe_decode(s, O.ptr(x), O.ptr(idx), O.ptr(w), 4,
                                           O.ptr(out))
            assert rc == 0, ghip.apus_ghip_last_error()
            outs[lim] = out
        want, eo = O.moe_forward(slabs, DIM, INTER, x, idx[None], w[None], limit=limit,
                                 want_expert_out=True)
        st = assert_close_combined(outs[limit], want[0],
                                   np.maximum(moe_floor(eo, w[None], idx[None])[0], inner[0]),
                                   "decode limit=%g trial %d" % (limit, trial))
        record("swiglu_limit%g_decode_trial%d" % (limit, trial), st, clamp_fracs=[round(float(v), 4) for v in frac])
        assert not np.array_equal(outs[limit], outs[10.0])


@pytest.mark.parametrize("T,k", [(40, 3), (600, 4)])
def test_prefill_clamps(store, slabs, T, k):
    ghip, stores, limit = store
    rng = np.random.default_rng(T * 7 + k)
    x = O.f32_to_bf16(rng.standard_normal((T, DIM)).astype(np.float32))
    idx, w = skewed_routing(rng, T, E, k, hot=2)
    inner, frac = oracle_inner(slabs, x, idx, w, limit)
    assert min(frac) > 0.05, frac
    outs = {lim: prefill(ghip, s, x, idx, w, host=(T < 100))
            for lim, s in stores.items()}
    want, eo = O.moe_forward(slabs, DIM, INTER, x, idx, w, limit=limit,
                             want_expert_out=True, threads=8)
    st = assert_close_combined(outs[limit], want, np.maximum(floor_of(eo, w, idx), inner),
                               "prefill limit=%g T=%d k=%d" % (limit, T, k))
    record("swiglu_limit%g_prefill_T%d_k%d" % (limit, T, k), st, clamp_fracs=[round(float(v), 4) for v in frac])
    assert not np.array_equal(outs[limit], outs[10.0])
