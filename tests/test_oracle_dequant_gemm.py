"""Pins of the oracle's dequant (c/fp8blk.h:115-136) and sequential-k
GEMV/GEMM (c/bf16.h:202-217, AVX2/mt legs c/bf16.h:444-767) — CPU only.

Checked against: the reference KATs (tests/m1/test_3_schema.py:87-103),
all 256 codes x scale corners in exact f64 arithmetic (tests/m3g/
test_m3g.c:135-179), an independent numpy sequential-k restatement, the
M-independence and thread-count invariants (tests/m3g/test_m3g.c:269-278,
Makefile:191-197), the golden fixtures written by the reference kernels,
and the reference build itself when present.
"""
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


def deq_exact_f64(codes, scales):
    """bf16_rne(f32(e4m3 * scale)): the e4m3 value has <= 4 significant bits
    and the scale 24, so the f64 product is exact; numpy's f32 cast is the
    single IEEE rounding; then RNE to bf16."""
    lut = np.array([O.lib().apo_e4m3_f32(c) for c in range(256)], np.float64)
    O_, K = codes.shape
    s = scales.astype(np.float64)[np.arange(O_)[:, None] // 128,
                                  np.arange(K)[None, :] // 128]
    p32 = (lut[codes] * s).astype(np.float32)
    return O.f32_to_bf16(p32)


def test_dequant_kats():
    codes = np.full((128, 256), 0x38, np.uint8)            # all 1.0
    out = O.dequant(codes, np.array([[2.0, 0.5]], np.float32))
    f = O.bf16_to_f32(out)
    assert np.all(f[:, :128] == 2.0) and np.all(f[:, 128:] == 0.5)
    codes = np.zeros((1, 128), np.uint8)
    codes[0, 0], codes[0, 1] = 0x01, 0xFE
    f = O.bf16_to_f32(O.dequant(codes, np.array([[4.0]], np.float32)))
    assert f[0, 0] == 2.0 ** -7 and f[0, 1] == -1792.0 and f[0, 2] == 0.0


SCALE_CORNERS = [1.0, 0.5, -2.0, 0.0, 2.0 ** -126, 2.0 ** -127, 2.0 ** 40,
                 448.0, 2.0 ** -9, 3.14159e-30]


@pytest.mark.parametrize("scale", SCALE_CORNERS)
def test_dequant_all_codes_scale_corners(scale):
    codes = np.array([[(o * 64 + k) & 0xFF for k in range(256)]
                      for o in range(4)], np.uint8)
    scales = np.full((1, 2), scale, np.float32)
    got = O.dequant(codes, scales)
    assert np.array_equal(got, deq_exact_f64(codes, scales))
    assert np.array_equal(O.dequant(codes, scales, threads=3), got)


def test_dequant_golden(fx, man):
    for i, sh in enumerate(man["dequant"]):
        codes, scales = fx[f"deq{i}_codes"], fx[f"deq{i}_scales"]
        want = fx[f"deq{i}_out"]
        assert np.array_equal(O.dequant(codes, scales), want), sh
        assert np.array_equal(O.dequant(codes, scales, threads=4), want), sh
        assert np.array_equal(deq_exact_f64(codes, scales), want), sh


def numpy_seq_gemm(w, x):
    """Independent restatement: fp32 accumulate over k ascending, vectorized
    over (m, o); every numpy f32 op is one IEEE rounding (no FMA)."""
    wf, xf = O.bf16_to_f32(w), O.bf16_to_f32(x)
    acc = np.zeros((x.shape[0], w.shape[0]), np.float32)
    for k in range(w.shape[1]):
        acc = acc + (xf[:, k:k + 1] * wf[None, :, k])
    return O.f32_to_bf16(acc)


def test_gemm_golden(fx, man):
    for i, sh in enumerate(man["gemm"]):
        w, x, want = fx[f"gem{i}_w"], fx[f"gem{i}_x"], fx[f"gem{i}_y"]
        assert np.array_equal(O.gemm(w, x), want), sh
        assert np.array_equal(O.gemm(w, x, threads=4), want), sh
        assert np.array_equal(numpy_seq_gemm(w, x), want), sh


def test_linear_golden(fx, man):
    for i, sh in enumerate(man["linear"]):
        got = O.fp8_linear(fx[f"lin{i}_codes"], fx[f"lin{i}_scales"],
                           fx[f"lin{i}_x"], threads=1)
        assert np.array_equal(got, fx[f"lin{i}_y"]), sh
        got = O.fp8_linear(fx[f"lin{i}_codes"], fx[f"lin{i}_scales"],
                           fx[f"lin{i}_x"], threads=5)
        assert np.array_equal(got, fx[f"lin{i}_y"]), sh


SWEEP = [(1, 1, 1), (1, 9, 17), (3, 5, 31), (2, 11, 32), (5, 12, 33),
         (4, 8, 63), (7, 16, 64), (1, 24, 65), (6, 13, 96), (2, 40, 127),
         (8, 17, 128), (3, 25, 129), (1, 100, 200), (5, 33, 257),
         (4, 64, 384), (2, 128, 96), (9, 7, 41), (1, 200, 37)]


def test_gemm_sweep_invariants():
    """tests/m3g/test_m3g.c:308-351 sweep: random finite bf16 codes; mt ==
    scalar at several thread counts; M-independence (row m == GEMV of m)."""
    rng = np.random.default_rng(0x12345)
    for (M, Oo, K) in SWEEP:
        w = rng.integers(0, 1 << 16, (Oo, K), dtype=np.uint32).astype(np.uint16)
        x = rng.integers(0, 1 << 16, (M, K), dtype=np.uint32).astype(np.uint16)
        w[(w & 0x7F80) == 0x7F80] = 0x3F80
        x[(x & 0x7F80) == 0x7F80] = 0x3F80
        y = O.gemm(w, x)
        for t in (2, 3, 8):
            assert np.array_equal(O.gemm(w, x, threads=t), y), (M, Oo, K, t)
        for m in range(M):
            assert np.array_equal(O.gemm(w, x[m:m + 1])[0], y[m]), (M, Oo, K, m)


def test_gemm_planted_order_mistake_is_detected():
    """A reordered sum (descending k) differs from the anchor on a case
    built to cancel: the sequential-k pin is not vacuous."""
    w = O.f32_to_bf16(np.array([[2.0 ** 30, 1.0, -2.0 ** 30, 1.0]], np.float32))
    x = O.f32_to_bf16(np.ones((1, 4), np.float32))
    y = O.bf16_to_f32(O.gemm(w, x))[0, 0]
    # ascending: ((2^30 + 1) - 2^30) + 1 = 1 (the first 1 is absorbed)
    assert y == 1.0
    # descending: ((1 - 2^30) + 1) + 2^30 = 0 (the second 1 is absorbed)
    rev = O.bf16_to_f32(O.gemm(w[:, ::-1].copy(), x))[0, 0]
    assert rev == 0.0


@pytest.mark.skipif(not O.ref_available(), reason="reference build absent")
def test_vs_reference_build_large():
    R = O.ref()
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 256, (1536, 4096), dtype=np.uint8)
    scales = np.exp2(rng.uniform(-12, -4, (12, 32))).astype(np.float32)
    x = O.f32_to_bf16(rng.standard_normal((5, 4096)).astype(np.float32))
    y_ref = np.empty((5, 1536), np.uint16)
    assert R.ref_fp8blk_linear_mt(O.ptr(codes), O.ptr(scales), O.ptr(x),
                                  O.ptr(y_ref), 5, 1536, 4096) == 0
    assert np.array_equal(O.fp8_linear(codes, scales, x, threads=8), y_ref)
    out_ref = np.empty((1536, 4096), np.uint16)
    R.ref_fp8blk_dequant_mt(O.ptr(codes), O.ptr(scales), O.ptr(out_ref), 1536, 4096)
    assert np.array_equal(O.dequant(codes, scales, threads=8), out_ref)
