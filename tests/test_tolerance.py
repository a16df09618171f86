"""The tolerance helpers themselves (CPU): bf16 ulp sizes, the ordered ulp
distance across zero, and the combined-output test at cancellation scale."""
import numpy as np

import oracle as O
from tolerance import bf16_ulp_at, compare, compare_combined


def test_ulp_at_powers_of_two():
    v = np.array([1.0, 1.5, 1.9921875, 0.75, 2.0 ** -20, 3e38, 0.0])
    want = np.array([2.0 ** -7, 2.0 ** -7, 2.0 ** -7, 2.0 ** -8, 2.0 ** -27,
                     2.0 ** 120, 0.0])
    assert np.array_equal(bf16_ulp_at(v), want)
    # the ulp of a bf16 value is the gap to its successor
    codes = np.array([0x3F80, 0x4049, 0x3E00, 0x7F00], np.uint16)
    x = O.bf16_to_f32(codes).astype(np.float64)
    nxt = O.bf16_to_f32(codes + np.uint16(1)).astype(np.float64)
    assert np.array_equal(bf16_ulp_at(x), nxt - x)


def test_ulp_distance_across_zero():
    a = np.array([0x0001, 0x8001, 0x0000, 0x8000], np.uint16)
    b = np.array([0x8001, 0x0001, 0x8000, 0x0000], np.uint16)
    st = compare(a, b, 1.0)
    assert st["max_ulp"] == 2 and st["frac_le1ulp"] == 0.5


def test_combined_scale():
    """A cancelling sum (|ref| << floor): one ulp of the floor's scale passes,
    three do not; identical outputs pass; a wrong term fails max_rel."""
    floor = np.full(4, 100.0)                     # ulp at 100 = 0.5
    ref = O.f32_to_bf16(np.array([0.25, -1.0, 3.0, 0.0], np.float32))
    one = O.f32_to_bf16(np.array([0.75, -1.5, 2.5, 0.5], np.float32))
    three = O.f32_to_bf16(np.array([1.75, -1.0, 3.0, 0.0], np.float32))
    assert compare_combined(ref, ref, floor)["frac_le1ulp_scaled"] == 1.0
    assert compare_combined(one, ref, floor)["frac_le1ulp_scaled"] == 1.0
    assert compare_combined(three, ref, floor)["frac_le1ulp_scaled"] == 0.75
    wrong = O.f32_to_bf16(np.array([20.25, -1.0, 3.0, 0.0], np.float32))
    assert compare_combined(wrong, ref, floor)["max_rel"] > 1e-2
