"""The shared synthetic generator (include/apus_synth.h): distribution
properties of the BASELINE.json inputs and sub-range reproducibility."""
import ctypes

import numpy as np

import oracle as O


def test_fp8_codes_finite_and_uniform(pkg):
    lib = pkg.load()
    n = 254 * 4000
    c = np.empty(n, np.uint8)
    lib.apus_synth_fp8_codes(O.ptr(c), n, 1, 10, 0)
    assert not np.any((c & 0x7F) == 0x7F)            # 0x7F / 0xFF excluded
    hist = np.bincount(c, minlength=256)
    assert np.count_nonzero(hist) == 254
    assert hist[hist > 0].min() > 3500 and hist.max() < 4500
    part = np.empty(1000, np.uint8)
    lib.apus_synth_fp8_codes(O.ptr(part), 1000, 1, 10, 5000)
    assert np.array_equal(part, c[5000:6000])          # counter-based


def test_scales_log_uniform(pkg):
    lib = pkg.load()
    s = np.empty(20000, np.float32)
    lib.apus_synth_scales(O.ptr(s), s.size, 2, 11, 1e-4, 1e-2)
    assert s.min() >= np.float32(1e-4) and s.max() <= np.float32(1e-2)
    l = np.log10(s.astype(np.float64))
    assert abs(l.mean() + 3.0) < 0.02 and abs(l.std() - 2 / np.sqrt(12)) < 0.02


def test_bf16_normal(pkg):
    lib = pkg.load()
    tab = np.empty(65536, np.uint16)
    lib.apus_synth_normal_table(O.ptr(tab))
    f = O.bf16_to_f32(tab)
    assert np.all(np.diff(f) >= 0)                     # quantiles ascend
    assert np.array_equal(f, -f[::-1])                 # symmetric
    x = np.empty(200000, np.uint16)
    lib.apus_synth_bf16_normal(O.ptr(x), x.size, 3, 12, 0)
    v = O.bf16_to_f32(x).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1) < 0.01


def test_route_zipf_and_uniform(pkg):
    lib = pkg.load()
    T, E, k = 2048, 288, 8
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    assert lib.apus_synth_route(O.ptr(idx), O.ptr(w), T, E, k,
                                ctypes.c_double(1.1), 7) == 0
    assert idx.min() >= 0 and idx.max() < E
    assert all(len(set(r)) == k for r in idx)          # distinct per token
    assert np.allclose(w.sum(1), 1.0, atol=1e-6) and (w > 0).all()
    m = np.bincount(idx.ravel(), minlength=E)
    assert m.max() > 300 and m.min() <= 5              # ragged (BASELINE cfg 3)
    assert lib.apus_synth_route(O.ptr(idx), O.ptr(w), T, E, k,
                                ctypes.c_double(0.0), 7) == 0
    m = np.bincount(idx.ravel(), minlength=E)
    assert m.min() > 20 and m.max() < 100              # uniform
