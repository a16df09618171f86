"""Pins of the oracle's codec (c/num.h:136-166) — CPU only.

E4M3 decode: the reference KATs of tests/m1/test_3_schema.py:62-85, the
closed form (8+m)*2^(e-10) / m*2^-9 evaluated with Python floats, all 256
codes, monotonicity. BF16 narrow: an independent nearest-even definition
(compare the two bf16 neighbours in exact f64 arithmetic), exhaustive
widen/narrow round trip (tests/m3g/test_m3g.c:97-112).
"""
import math
import struct

import numpy as np
import pytest


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def closed_form(c):
    e, m = (c >> 3) & 15, c & 7
    v = math.ldexp(8 + m, e - 10) if e else math.ldexp(m, -9)
    return -v if c & 0x80 else v


def test_e4m3_kats(orc):
    L = orc.lib()
    kat = {0x00: 0.0, 0x38: 1.0, 0x30: 0.5, 0x40: 2.0, 0xC0: -2.0,
           0x7E: 448.0, 0xFE: -448.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9}
    for c, v in kat.items():
        assert L.apo_e4m3_f32(c) == v, hex(c)
    assert math.copysign(1.0, L.apo_e4m3_f32(0x80)) < 0          # -0
    # NaN codes decode as +-480 (c/num.h:136-141, c/fp8blk.h:18-21)
    assert L.apo_e4m3_f32(0x7F) == 480.0
    assert L.apo_e4m3_f32(0xFF) == -480.0


def test_e4m3_all_codes_closed_form(orc):
    L = orc.lib()
    for c in range(256):
        got = L.apo_e4m3_f32(c)
        assert f32_bits(got) == f32_bits(closed_form(c)), hex(c)


def test_e4m3_monotonic(orc):
    L = orc.lib()
    pos = [L.apo_e4m3_f32(c) for c in range(0x00, 0x7F)]
    neg = [L.apo_e4m3_f32(c) for c in range(0x80, 0xFF)]
    assert pos == sorted(pos) and len(set(pos)) == len(pos)
    assert neg == sorted(neg, reverse=True)


def _mag_value(bits):
    """Exact value of a non-negative f32 bit pattern, with the exponent
    field 255 read as the unbounded next binade (2^128 for the overflow
    candidate)."""
    e, m = (bits >> 23) & 0xFF, bits & 0x7FFFFF
    if e == 0:
        return math.ldexp(m, -149)
    return math.ldexp(m | 0x800000, e - 150)


def rne_reference(x32):
    """Nearest bf16 to an f32 value, ties to even, by comparing the two
    bf16 neighbours of |x| in exact f64 arithmetic (independent of the
    add-0x7FFF bit trick). Overflow past the largest bf16 gives inf."""
    u = f32_bits(x32)
    sign, mag = u & 0x80000000, u & 0x7FFFFFFF
    lo = mag & 0xFFFF0000
    hi = lo + 0x10000
    x, flo, fhi = _mag_value(mag), _mag_value(lo), _mag_value(hi)
    if x - flo < fhi - x:
        r = lo
    elif fhi - x < x - flo:
        r = hi
    else:
        r = lo if ((lo >> 16) & 1) == 0 else hi
    return (sign | r) >> 16


def test_bf16_narrow_vs_nearest_even(orc):
    L = orc.lib()
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32)
    # add exact ties and near-ties around several exponents
    base = rng.integers(0, 1 << 16, 2000, dtype=np.uint32) << 16
    extra = np.concatenate([base | 0x8000, base | 0x7FFF, base | 0x8001,
                            np.array([0x7F7FFFFF, 0x7F7F8000, 0x00008000,
                                      0x80008000, 0x00000001], np.uint32)])
    for u in np.concatenate([bits, extra]):
        u = int(u)
        if (u & 0x7FFFFFFF) > 0x7F800000:
            # NaN passes through as its high half; quiet NaNs only, since a
            # signalling NaN is quieted by the f32->double->f32 ctypes trip
            u |= 0x00400000
            assert L.apo_bf16_bits(struct.unpack("<f", struct.pack("<I", u))[0]) == u >> 16
            continue
        x = struct.unpack("<f", struct.pack("<I", u))[0]
        assert L.apo_bf16_bits(x) == rne_reference(x), hex(u)


def test_bf16_roundtrip_exhaustive(orc):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = orc.bf16_to_f32(codes)
    assert np.array_equal(f.view(np.uint32), codes.astype(np.uint32) << 16)
    L = orc.lib()
    nan = (codes & 0x7FFF) > 0x7F80
    for c in codes[::97]:
        assert L.apo_bf16_bits(float(orc.bf16_to_f32(np.array([c]))[0])) == c \
            or nan[c]


@pytest.mark.skipif(not __import__("oracle").ref_available(),
                    reason="reference CPU kernels not built here")
def test_codec_vs_reference_build(orc):
    L, R = orc.lib(), orc.ref()
    for c in range(256):
        assert f32_bits(L.apo_e4m3_f32(c)) == f32_bits(R.ref_e4m3_f32(c))
    rng = np.random.default_rng(3)
    for u in rng.integers(0, 1 << 32, 5000, dtype=np.uint64):
        x = struct.unpack("<f", struct.pack("<I", int(u)))[0]
        assert L.apo_bf16_bits(x) == R.ref_bf16_bits(x)
