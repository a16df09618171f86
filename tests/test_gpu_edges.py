"""The reference GPU gate's edge battery (tests/m7b/test_gkernels.c:215-279)
on both hooks, at the GEMV row counts (M = 1: the streaming MFMA GEMV) and at
GEMM row counts (M >= 16: the MFMA GEMM of the fp8blk_linear hook, the
grouped GEMV of the bf16_gemm hook), against the oracle's sequential-k
result (c/bf16.h:202-217, pinned to the reference build):

  - all-zero weight rows and the zero rows around them: bitwise;
  - +-inf weights against a zero activation (0 * inf) and inf - inf: NaN,
    bitwise: the x86 reference's default NaN (0xFFC00000, bf16 0xFFC0) is
    also what the MFMA units produce for 0 * inf and inf - inf;
  - an inf activation against finite weights: +-inf bitwise;
  - rows of pure bf16-subnormal weights: every product is fp32-subnormal,
    the denormal-flush class of the reference's own GPU gate, bounded by
    1e-37 (test_gkernels.c:257-266);
  - the fp32-subnormal accumulator probe (products ~2^-266): bound 1e-38;
  - mixed subnormal + normal rows and the random rows: the GEMM tolerance.

A separate probe records whether the MFMA units flush bf16-subnormal
INPUTS (a subnormal weight times 2^100 is a normal fp32 product): the
result is printed and recorded; either behavior is within the flush class.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from tolerance import assert_close, record, bf16_f32

pytestmark = pytest.mark.gpu

INF, NINF, SUB, NSUB = 0x7F80, 0xFF80, 0x0001, 0x8001


def is_nan(b):
    b = np.asarray(b, np.uint16)
    return ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)


def check_classes(got, want, cls, floor, what):
    """cls per output element: 'bit', 'nan', 'flush37', 'flush38', 'tol'."""
    got = np.asarray(got, np.uint16).ravel()
    want = np.asarray(want, np.uint16).ravel()
    cls = np.asarray(cls).ravel()
    floor = np.asarray(floor, np.float64).ravel()
    m = cls == "bit"
    bad = np.nonzero(m & (got != want))[0]
    assert bad.size == 0, "%s: bitwise rows differ at %s (gpu %s ref %s)" % (
        what, bad[:8].tolist(), [hex(v) for v in got[bad[:8]]], [hex(v) for v in want[bad[:8]]])
    m = cls == "nan"
    assert np.all(is_nan(want[m])), "%s: oracle not NaN where expected" % what
    assert np.all(is_nan(got[m])), "%s: GPU not NaN at %s" % (
        what, np.nonzero(m & ~is_nan(got))[0][:8].tolist())
    bad = np.nonzero(m & (got != want))[0]
    assert bad.size == 0, "%s: NaN payloads differ (gpu %s ref %s)" % (
        what, [hex(v) for v in got[bad[:4]]], [hex(v) for v in want[bad[:4]]])
    with np.errstate(invalid="ignore"):
        d = np.abs(bf16_f32(got).astype(np.float64) - bf16_f32(want).astype(np.float64))
    for c, bound in (("flush37", 1e-37), ("flush38", 1e-38)):
        m = cls == c
        if m.any():
            assert d[m].max() <= bound, "%s: %s class |d| %g > %g" % (what, c, d[m].max(), bound)
    m = cls == "tol"
    st = assert_close(got[m], want[m], floor[m], what + " (tolerance rows)")
    out = {"bitwise": int((cls == "bit").sum()), "nan": int((cls == "nan").sum()),
           "flush_max_abs": float(d[(cls == "flush37") | (cls == "flush38")].max())
           if ((cls == "flush37") | (cls == "flush38")).any() else 0.0,
           "nan_payloads_gpu": sorted({hex(v) for v in got[cls == "nan"]}),
           "nan_payloads_ref": sorted({hex(v) for v in want[cls == "nan"]})}
    out.update({"tol_" + k: v for k, v in st.items()})
    return out


def bf16_edge_case(rng, M):
    """test_gkernels.c:222-239 at M rows: O = 64, K = 256; rows 1-3 +-inf,
    4/5 pure subnormal, 6 mixed subnormal/normal, 0 and 7+ zero; x[:, 0] = 0."""
    Oo, K = 64, 256
    w = np.zeros((Oo, K), np.uint16)
    k = np.arange(K)
    w[1], w[2] = INF, NINF
    w[3] = np.where(k & 1, INF, NINF)
    w[4], w[5] = SUB, NSUB
    w[6] = np.where(k & 1, SUB, O.f32_to_bf16(rng.uniform(-2, 2, K).astype(np.float32)))
    x = O.f32_to_bf16(rng.uniform(-2, 2, (M, K)).astype(np.float32))
    x[:, 0] = 0
    cls = np.full((M, Oo), "bit", object)
    cls[:, 1:4] = "nan"
    cls[:, 4:6] = "flush37"
    cls[:, 6] = "tol"
    return w, x, cls


def run_bf16(ghip, w, x, via_hook=False):
    Oo, K = w.shape
    M = x.shape[0]
    y = np.empty((M, Oo), np.uint16)
    if via_hook:
        hooks = (ctypes.c_void_p * 2).in_dll(ghip, "apus_ghip_hooks")
        fn = ctypes.CFUNCTYPE(ctypes.c_int, *([ctypes.c_void_p] * 3 + [ctypes.c_size_t] * 3))(
            hooks[0])
        rc = fn(O.ptr(w), O.ptr(x), O.ptr(y), M, Oo, K)
    else:
        rc = ghip.apus_ghip_bf16_gemm(O.ptr(w), O.ptr(x), O.ptr(y), M, Oo, K)
    assert rc == 0, ghip.apus_ghip_last_error()
    return y


@pytest.mark.parametrize("M,via_hook", [(1, False), (1, True), (16, False), (17, True)])
def test_bf16_edges(ghip, M, via_hook):
    rng = np.random.default_rng(0xED + M)
    w, x, cls = bf16_edge_case(rng, M)
    want = O.gemm(w, x)
    got = run_bf16(ghip, w, x, via_hook)
    with np.errstate(invalid="ignore", over="ignore"):
        fl = 2.0 ** -8 * O.absdot(w, x)
    st = check_classes(got, want, cls, fl, "bf16 edges M=%d" % M)
    assert np.all(is_nan(got[:, 1:4]))
    print("bf16 edges M=%d" % M, st)
    record("edges_bf16_M%d%s" % (M, "_hook" if via_hook else ""), st)


def test_bf16_fp32_subnormal_probe(ghip):
    """test_gkernels.c:268-278: w = x = the smallest bf16 subnormal, so every
    product (2^-266) underflows fp32."""
    K = 256
    w = np.full((1, K), SUB, np.uint16)
    x = np.full((1, K), SUB, np.uint16)
    want = O.gemm(w, x)
    got = run_bf16(ghip, w, x)
    d = abs(float(bf16_f32(got)[0, 0]) - float(bf16_f32(want)[0, 0]))
    print("fp32-subnormal probe: ref %s gpu %s" % (hex(want[0, 0]), hex(got[0, 0])))
    record("edges_bf16_fp32_subnormal_probe", {"ref": hex(want[0, 0]), "gpu": hex(got[0, 0]),
                                               "abs_diff": d})
    assert got[0, 0] == want[0, 0] or d <= 1e-38


@pytest.mark.parametrize("M", [1, 16])
def test_mfma_subnormal_input_probe(ghip, M):
    """Does the MFMA flush a bf16-subnormal input? Row 0: weights 2^-127
    (subnormal), row 1: 2^-126 (the smallest normal), x = 2^100: the exact
    products are the normal fp32 values 2^-27 and 2^-26, so row 0 is
    256 * 2^-27 = 2^-19 unless the subnormal input is flushed (then 0).
    Either outcome is inside the flush class (|d| <= 2^-19 ~ 1.9e-6 here
    only because x is huge; on normative data the class is ~1e-37)."""
    K = 256
    w = np.zeros((16, K), np.uint16)
    w[0], w[1] = 0x0040, 0x0080
    x = np.full((M, K), 0x7180, np.uint16)            # 2^100
    want = O.gemm(w, x)
    got = run_bf16(ghip, w, x)
    assert np.all(got[:, 1] == want[:, 1]), (hex(got[0, 1]), hex(want[0, 1]))   # 2^-18
    flushed = bool(np.all(got[:, 0] == 0))
    exact = bool(np.all(got[:, 0] == want[:, 0]))
    print("MFMA bf16 subnormal input (M=%d): %s (gpu %s, ref %s)" % (
        M, "flushed to zero" if flushed else "kept" if exact else "other",
        hex(got[0, 0]), hex(want[0, 0])))
    record("mfma_bf16_subnormal_input_M%d" % M,
           {"behavior": "flushed" if flushed else "kept" if exact else "other",
            "gpu": hex(got[0, 0]), "ref": hex(want[0, 0])})
    assert flushed or exact


def fp8_edge_case(rng, M, inf=True):
    """The fp8blk_linear counterpart: codes cannot be inf, so the inf comes
    from the activation. O = 256, K = 256 (the MFMA GEMM's shapes at M >= 16).
    Block row 0 (rows 0-127) has normal scales: row 0 all-zero codes, row 1
    code 1.0 at k = 0 only, row 2 codes +1.0 / -1.0 at k = 0 / 1, rows 3+
    random. Block row 1 (rows 128-255): scale 2^-141 on k block 0 (bf16
    subnormal weights, |w| <= 448 * 2^-141, so with |x| < ~4 every product
    is fp32-subnormal and a row sums to < 1e-37, the reference's class) and
    normal on k block 1; rows 128-131 have zero codes in k block 1 (pure
    subnormal rows). With inf, x[0, 0] = x[0, 1] = +inf
    (inf - inf where the two weights differ in sign, as in row 2); every
    other activation is normal."""
    Oo, K = 256, 256
    codes = rng.integers(0, 254, (Oo, K), dtype=np.uint8)
    codes[codes >= 0x7F] += 1                       # finite codes only
    codes[0] = 0
    codes[1] = 0
    codes[1, 0] = 0x38
    codes[2] = 0
    codes[2, 0], codes[2, 1] = 0x38, 0xB8
    codes[128:132, 128:] = 0
    scales = np.array([[1e-3, 2e-3], [2.0 ** -141, 1e-3]], np.float32)
    x = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    cls = np.full((M, Oo), "tol", object)
    cls[:, 0] = "bit"                                     # zero codes -> +0
    cls[:, 128:132] = "flush37"
    if not inf:
        return codes, scales, x, cls
    x[0, 0] = x[0, 1] = INF
    deq = O.dequant(codes, scales)
    # row 0 of x (the inf activations): NaN where a weight at k=0 or 1 is
    # zero (0 * inf) or the two inf terms cancel, else +-inf (bitwise)
    w0, w1 = bf16_f32(deq[:, 0]), bf16_f32(deq[:, 1])
    with np.errstate(invalid="ignore"):
        nan_row = (w0 == 0) | (w1 == 0) | (np.sign(w0) != np.sign(w1))
    cls[0] = np.where(nan_row, "nan", "bit")
    return codes, scales, x, cls


def run_fp8(ghip, codes, scales, x, via_hook=False):
    Oo, K = codes.shape
    M = x.shape[0]
    y = np.empty((M, Oo), np.uint16)
    if via_hook:
        hooks = (ctypes.c_void_p * 2).in_dll(ghip, "apus_ghip_hooks")
        fn = ctypes.CFUNCTYPE(ctypes.c_int, *([ctypes.c_void_p] * 4 + [ctypes.c_size_t] * 3))(
            hooks[1])
        rc = fn(O.ptr(codes), O.ptr(scales), O.ptr(x), O.ptr(y), M, Oo, K)
    else:
        rc = ghip.apus_ghip_fp8blk_linear(O.ptr(codes), O.ptr(scales), O.ptr(x), O.ptr(y),
                                          M, Oo, K)
    assert rc == 0, ghip.apus_ghip_last_error()
    return y


@pytest.mark.parametrize("M,inf,via_hook", [(1, True, False), (1, False, True),
                                            (16, True, False), (32, True, True)])
def test_fp8_edges(ghip, M, inf, via_hook):
    rng = np.random.default_rng(0xE8 + M)
    codes, scales, x, cls = fp8_edge_case(rng, M, inf)
    want = O.fp8_linear(codes, scales, x)
    got = run_fp8(ghip, codes, scales, x, via_hook)
    with np.errstate(invalid="ignore", over="ignore"):
        fl = 2.0 ** -8 * O.absdot(O.dequant(codes, scales), x)
    st = check_classes(got, want, cls, fl, "fp8 edges M=%d" % M)
    print("fp8 edges M=%d" % M, st)
    record("edges_fp8_M%d%s%s" % (M, "_inf" if inf else "", "_hook" if via_hook else ""), st)
