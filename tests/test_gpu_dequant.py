"""K1 on the GPU: FP8-block dequant must be BITWISE equal to the oracle
(c/fp8blk.h:115-136) — fast decode on every finite code, exact decode on
all 256 codes, across the scale corners of tests/m3g/test_m3g.c:135-179,
ceil shapes and the BASELINE config-0 matrix."""
import ctypes
import json
import os

import numpy as np
import pytest

import oracle as O
import gpu_util as G

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")

SCALES = [1.0, 0.5, -2.0, 0.0, 2.0 ** -126, 2.0 ** -127, 2.0 ** 40, 448.0,
          2.0 ** -9, 3.14159e-30, 1e-4, 1e-2]


def gpu_dequant_dev(ghip, codes, scales, exact):
    O_, K = codes.shape
    dc, ds = G.dev(codes), G.dev(scales)
    out = G.empty(O_ * K * 2)
    rc = ghip.apus_ghip_fp8blk_dequant_dev(G.vp(dc), G.vp(ds), G.vp(out), O_, K,
                                           exact, G.stream())
    assert rc == 0
    return G.host(out, np.uint16, (O_, K))


@pytest.mark.parametrize("scale", SCALES)
def test_all_codes_scale_corners(ghip, scale):
    codes = np.array([[(o * 64 + k) & 0xFF for k in range(256)] for o in range(4)],
                     np.uint8)
    scales = np.full((1, 2), scale, np.float32)
    want = O.dequant(codes, scales)
    got = gpu_dequant_dev(ghip, codes, scales, 1)
    assert np.array_equal(got, want), "exact decode, scale %r" % scale
    finite = codes.copy()
    finite[(finite & 0x7F) == 0x7F] = 0x00
    want_f = O.dequant(finite, scales)
    got_f = gpu_dequant_dev(ghip, finite, scales, 0)
    bad = np.argwhere(got_f != want_f)
    assert bad.size == 0, "fast decode, scale %r: %d mismatches, first code %#x" % (
        scale, len(bad), finite[tuple(bad[0])] if bad.size else 0)


def test_golden_shapes_host_entry(ghip):
    fx = np.load(os.path.join(GOLD, "fixtures.npz"))
    man = json.load(open(os.path.join(GOLD, "manifest.json")))
    for i, sh in enumerate(man["dequant"]):
        codes, scales = fx[f"deq{i}_codes"], fx[f"deq{i}_scales"]
        out = np.empty(codes.shape, np.uint16)
        rc = ghip.apus_ghip_fp8blk_dequant(O.ptr(codes), O.ptr(scales), O.ptr(out),
                                           *codes.shape)
        assert rc == 0
        assert np.array_equal(out, fx[f"deq{i}_out"]), sh
        if codes.shape[1] % 16 == 0:
            assert np.array_equal(gpu_dequant_dev(ghip, codes, scales, 0),
                                  fx[f"deq{i}_out"]), ("fast", sh)


def test_config0_matrix_fast_path(ghip, pkg):
    lib = pkg.load()
    N, K = 2048, 4096
    codes = np.empty((N, K), np.uint8)
    lib.apus_synth_fp8_codes(O.ptr(codes), codes.size, 0xC0, 10, 0)
    scales = np.empty((16, 32), np.float32)
    lib.apus_synth_scales(O.ptr(scales), scales.size, 0xC0, 11, 1e-4, 1e-2)
    want = O.dequant(codes, scales, threads=8)
    assert np.array_equal(gpu_dequant_dev(ghip, codes, scales, 0), want)
    assert np.array_equal(gpu_dequant_dev(ghip, codes, scales, 1), want)


def test_device_synth_matches_host(ghip, pkg):
    lib = pkg.load()
    n = 1 << 20
    h = np.empty(n + 5, np.uint8)
    lib.apus_synth_fp8_codes(O.ptr(h), h.size, 9, 77, 3)
    d = G.empty(h.size)
    assert lib.apus_synth_fp8_codes_dev(G.vp(d), h.size, 9, 77, 3, G.stream()) == 0
    assert np.array_equal(G.host(d, np.uint8, h.shape), h)
    hb = np.empty(100003, np.uint16)
    lib.apus_synth_bf16_normal(O.ptr(hb), hb.size, 9, 78, 11)
    db = G.empty(hb.size * 2)
    assert lib.apus_synth_bf16_normal_dev(G.vp(db), hb.size, 9, 78, 11, G.stream()) == 0
    assert np.array_equal(G.host(db, np.uint16, hb.shape), hb)
