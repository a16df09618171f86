"""Size-independent properties at the BASELINE shapes, checked bitwise on the
GPU (no oracle needed at these sizes):

- config 1 (dense FP8 GEMV, W [16384, 4096], M = 1, 2, 4, and the GEMM
  path at M = 16): scaling x by a power of two
  scales every product, partial sum and rounding by the same power, so
  y(2^-4 x) * 2^4 == y(x) element for element wherever nothing is subnormal;
- config 2 (MoE decode, 288 experts, top-8): the combine runs in ascending
  expert order (c/gmoe.h:307-320), so the order of the routing slots does
  not change a bit of the output;
- config 3 (prefill, T = 2048, Zipf(1.1)): each token's output depends only
  on its own row and routing (c/gmoe.h:278-320 loops over tokens), so
  permuting the tokens permutes the output rows, bitwise, although the
  permuted pairs land in other rows of other tiles of the grouped GEMMs.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import gpu_util as G

pytestmark = pytest.mark.gpu

E, DIM, INTER = 288, 4096, 2048


def open_store(ghip, E, dim, inter, limit=10.0):
    s = ctypes.c_void_p()
    err = ctypes.create_string_buffer(256)
    assert ghip.apus_ghip_store_open(ctypes.byref(s), E, dim, inter, limit, err,
                                     256) == 0, err.value
    return s


def test_config1_power_of_two_scaling(ghip, pkg):
    lib = pkg.load()
    N, K = 16384, 4096
    codes = np.empty((N, K), np.uint8)
    lib.apus_synth_fp8_codes(O.ptr(codes), codes.size, 0xC1, 10, 0)
    sc = np.empty((N // 128, K // 128), np.float32)
    lib.apus_synth_scales(O.ptr(sc), sc.size, 0xC1, 11, 1e-4, 1e-2)
    x = np.empty((16, K), np.uint16)
    lib.apus_synth_bf16_normal(O.ptr(x), x.size, 0xC1, 12, 0)
    xs = O.f32_to_bf16(O.bf16_to_f32(x) * np.float32(2.0 ** -4))
    assert np.array_equal(O.bf16_to_f32(xs) * np.float32(16.0), O.bf16_to_f32(x))
    dc, ds = G.dev(codes), G.dev(sc)
    for M in (1, 2, 4, 16):                   # streaming GEMV, then the MFMA GEMM
        outs = []
        for xin in (x, xs):
            dx, dy = G.dev(xin[:M]), G.empty(M * N * 2)
            assert ghip.apus_ghip_fp8blk_linear_dev(G.vp(dc), G.vp(ds), G.vp(dx), G.vp(dy),
                                                   M, N, K, 0, None) == 0
            outs.append(O.bf16_to_f32(G.host(dy, np.uint16, (M, N))))
        y, ys = outs
        ok = np.abs(y) > 2.0 ** -100          # scaled value stays normal
        assert ok.mean() > 0.99
        assert np.array_equal((ys * np.float32(16.0))[ok], y[ok]), "M=%d" % M


def test_config2_slot_order_invariant(ghip, pkg):
    lib = pkg.load()
    k, seed = 8, 0xC2
    s = open_store(ghip, E, DIM, INTER)
    try:
        assert ghip.apus_ghip_store_synth(s, seed, 0, 1e-4, 1e-2) == 0
        logits = np.empty(E, np.float32)
        lib.apus_synth_f32_normal(O.ptr(logits), E, seed, 50, 0)
        x = np.empty(DIM, np.uint16)
        lib.apus_synth_bf16_normal(O.ptr(x), DIM, seed, 51, 0)
        idx, w = O.route_softmax(logits, k)
        idx = np.ascontiguousarray(idx, np.int32)
        w = np.ascontiguousarray(w, np.float32)
        dx = G.dev(x)

        def run(ii, ww):
            di, dw, do = G.dev(ii), G.dev(ww), G.empty(DIM * 2)
            assert ghip.apus_ghip_moe_decode_dev(s, G.vp(dx), None, G.vp(di), G.vp(dw), k,
                                                 G.vp(do), G.stream()) == 0
            return G.host(do, np.uint16, (DIM,))

        ref = run(idx, w)
        assert np.abs(O.bf16_to_f32(ref)).max() > 0
        rng = np.random.default_rng(5)
        for p in [np.arange(k)[::-1]] + [rng.permutation(k) for _ in range(3)]:
            got = run(np.ascontiguousarray(idx[p]), np.ascontiguousarray(w[p]))
            assert np.array_equal(got, ref), "slot order %s" % p.tolist()
    finally:
        ghip.apus_ghip_store_close(s)


@pytest.mark.timeout(300)
def test_config3_token_permutation_equivariant(ghip, pkg):
    lib = pkg.load()
    k, T, seed = 8, 2048, 0xC3
    s = open_store(ghip, E, DIM, INTER)
    try:
        assert ghip.apus_ghip_store_synth(s, seed, 0, 1e-4, 1e-2) == 0
        idx = np.empty((T, k), np.int32)
        w = np.empty((T, k), np.float32)
        assert lib.apus_synth_route(O.ptr(idx), O.ptr(w), T, E, k, 1.1, seed) == 0
        x = np.empty((T, DIM), np.uint16)
        lib.apus_synth_bf16_normal(O.ptr(x), x.size, seed, 52, 0)

        def run(xx, ii, ww):
            dx, di, dw = G.dev(xx), G.dev(ii), G.dev(ww)
            do = G.empty(T * DIM * 2)
            assert ghip.apus_ghip_moe_prefill_dev(s, G.vp(dx), T, G.vp(di), G.vp(dw), k,
                                                  G.vp(do), G.stream()) == 0
            return G.host(do, np.uint16, (T, DIM))

        ref = run(x, idx, w)
        p = np.random.default_rng(6).permutation(T)
        got = run(np.ascontiguousarray(x[p]), np.ascontiguousarray(idx[p]),
                  np.ascontiguousarray(w[p]))
        bad = np.nonzero((got != ref[p]).any(1))[0]
        assert bad.size == 0, "%d of %d permuted rows differ (first %s)" % (
            bad.size, T, bad[:5].tolist())
    finally:
        ghip.apus_ghip_store_close(s)
