"""Pins the 8-bit K/V oracle (oracle/kv8.py) on the CPU."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import kv8


def test_hand_computed_rows():
    # absmax 127 -> scale exactly 1: the values themselves, ties to even.
    q, s = kv8.quantize(np.array([[127.0, -63.5, 0.5, 1.5, -2.5, 3.0]]))
    assert float(s[0]) == 1.0
    assert q[0].tolist() == [127, -64, 0, 2, -2, 3]
    # absmax 254 -> scale 2.
    q, s = kv8.quantize(np.array([[254.0, 1.0, 3.0, -5.0]]))
    assert float(s[0]) == 2.0 and q[0].tolist() == [127, 0, 2, -2]
    # An all-zero row takes the 1e-4 floor and stays zero.
    q, s = kv8.quantize(np.zeros((1, 8)))
    assert float(s[0]) == float(np.float16(np.float32(1e-4) / np.float32(127)))
    assert not q.any()
    assert q.dtype == np.int8 and s.dtype == np.float16


def test_fp16_rounding_of_the_scale_can_clip_the_maximum():
    """The scale is rounded to fp16 before the division, so the largest
    element can land on 127.x and is clipped (paged_kv.py:53-55)."""
    x = np.array([[1.0, 0.3]], dtype=np.float32)
    scale = np.float16(np.float32(1.0) / np.float32(127.0))
    q, s = kv8.quantize(x)
    assert s[0] == scale
    assert q[0, 0] == np.clip(np.rint(np.float32(1.0) / np.float32(scale)), -127, 127)
    assert abs(int(q[0, 0])) <= 127


@pytest.mark.parametrize("shape", [(5, 3, 128), (2, 1, 64), (7, 4, 80)])
def test_round_trip_error_is_half_a_step(shape):
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * rng.uniform(0.01, 10, shape[:-1])[..., None]).astype(np.float16)
    q, s = kv8.quantize(x)
    err = np.abs(x.astype(np.float32) - kv8.dequantize(q, s))
    bound = s.astype(np.float32)[..., None] * 0.5 * (1 + 1e-3)
    # Clipping of the maximum (fp16-rounded scale) adds at most one more step.
    assert np.all(err <= bound + (np.abs(q) == 127) * s.astype(np.float32)[..., None])
    assert np.abs(q).max() <= 127


def test_scale_invariance_and_brute_force():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 16)).astype(np.float32)
    q1, s1 = kv8.quantize(x)
    q2, s2 = kv8.quantize(x * 4)  # a power of two scales exactly
    assert np.array_equal(q1, q2) and np.array_equal(s1.astype(np.float32) * 4, s2.astype(np.float32))
    for row, qrow, srow in zip(x, q1, s1):
        want, scale = kv8.quantize_brute(row)
        assert qrow.tolist() == want and float(srow) == scale


def _round_to_f16(value):
    """A Fraction rounded half to even to the nearest fp16 (finite range),
    from the fp16 grid alone."""
    from fractions import Fraction

    if value == 0:
        return 0.0
    sign = -1 if value < 0 else 1
    mag = abs(value)
    # fp16: 10 fraction bits, exponents -14..15, subnormal step 2^-24.
    exp = max(-14, min(15, mag.numerator.bit_length() - mag.denominator.bit_length()))
    while exp > -14 and Fraction(2) ** exp > mag:
        exp -= 1
    while exp < 15 and Fraction(2) ** (exp + 1) <= mag:
        exp += 1
    step = Fraction(2) ** (exp - 10)
    k, rem = divmod(mag, step)
    k = int(k)
    if rem * 2 > step or (rem * 2 == step and k % 2 == 1):
        k += 1
    return sign * float(k * step)


def test_gather_dequantize_is_one_rounding_of_the_exact_product():
    """Every int8 value times normal and subnormal fp16 scales: the float32
    product cast to fp16 (paged_kv.py:289-291) equals the exact rational
    product rounded half to even to fp16."""
    from fractions import Fraction

    q = np.arange(-127, 128, dtype=np.int8)
    scales = np.array([1e-4 / 127, 3e-6, 6.1e-5, 0.0078125, 0.01234, 0.5, 1.0, 3.3, 200.0],
                      dtype=np.float16)
    got = kv8.gather_dequantize(np.repeat(q[None, :], len(scales), axis=0), scales)
    for i, s in enumerate(scales):
        exact = [_round_to_f16(Fraction(int(b)) * Fraction(float(s))) for b in q]
        np.testing.assert_array_equal(got[i].astype(np.float64), np.array(exact))
