"""Pins the oracle's fp16 conversions and exact-dot rounding against numpy
(IEEE round-to-nearest-even) and exact rational arithmetic."""
from fractions import Fraction

import numpy as np


def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ours = orc.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(ours[np.isnan(ref)]))
    assert np.array_equal(ours[np.isinf(ref)], ref[np.isinf(ref)])


def _f32_cases():
    rng = np.random.default_rng(0)
    vals = [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-8, 1e-5, 1e-3, 1.0, 100.0, 6e4)]
    bits16 = np.arange(0, 0x7C00, dtype=np.uint32)
    # exact fp16 values, their midpoints and the neighbours of the midpoints
    h = bits16.astype(np.uint16).view(np.float16).astype(np.float64)
    hn = (bits16 + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((h + hn) / 2).astype(np.float32)
    mid_bits = mid.view(np.uint32)
    near = [mid, (mid_bits + 1).view(np.float32), (mid_bits - 1).view(np.float32), h.astype(np.float32)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e10, 5.96e-8, 2.98e-8, 2.9802322e-8, 1e-30,
                     np.inf, -np.inf], dtype=np.float32)
    allv = np.concatenate(vals + near + [edge, -np.concatenate(near)])
    return allv


def test_f32_to_f16_matches_numpy(orc):
    v = _f32_cases()
    ours = orc.f32_to_f16_bits(v)
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).view(np.uint16)
    nan = np.isnan(v)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(ours[nan].view(np.float16)))  # NaN payloads are not compared


def test_f64_to_f16_matches_numpy(orc):
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(200000) * s for s in (1e-7, 1e-3, 1.0, 3e4)])
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    hn = (np.arange(0, 0x7C00, dtype=np.uint32) + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = (h + hn) / 2
    v = np.concatenate([v, mid, np.nextafter(mid, 0), np.nextafter(mid, 1e9), -mid])
    ours = orc.f64_to_f16_bits(v)
    ref = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def _exact_dot(a16, b16, bias16=None):
    a = a16.view(np.float16).astype(np.float64)
    b = b16.view(np.float16).astype(np.float64)
    s = sum((Fraction(float(x)) * Fraction(float(y)) for x, y in zip(a, b)), Fraction(0))
    if bias16 is not None:
        s += Fraction(float(np.uint16(bias16).view(np.float16)))
    return s


def test_exact_dot_fix48_matches_fractions(orc):
    rng = np.random.default_rng(2)
    for n in (1, 2, 7, 64, 300):
        for scale in (1e-3, 1.0, 200.0):
            a = (rng.standard_normal(n) * scale).astype(np.float16).view(np.uint16)
            b = (rng.standard_normal(n) * scale).astype(np.float16).view(np.uint16)
            bias = np.float16(rng.standard_normal()).view(np.uint16)
            v = orc.dot_exact_fix48(a, b, int(bias))
            assert Fraction(v, 1 << 48) == _exact_dot(a, b, bias)


def test_exact_dot_extremes(orc):
    big = np.array([65504.0] * 1000, dtype=np.float16).view(np.uint16)
    tiny = np.array([2.0 ** -24] * 1000, dtype=np.float16).view(np.uint16)
    assert Fraction(orc.dot_exact_fix48(big, big), 1 << 48) == 1000 * Fraction(65504) ** 2
    assert Fraction(orc.dot_exact_fix48(tiny, tiny), 1 << 48) == 1000 * Fraction(1, 1 << 48)
    mixed_a = np.array([65504.0, 2.0 ** -24, -65504.0], dtype=np.float16).view(np.uint16)
    mixed_b = np.array([65504.0, 2.0 ** -24, 65504.0], dtype=np.float16).view(np.uint16)
    # big terms cancel exactly, the tiny product survives
    assert orc.dot_exact_fix48(mixed_a, mixed_b) == 1


def test_fix48_rounding_against_numpy_when_double_exact(orc):
    rng = np.random.default_rng(3)
    for _ in range(4000):
        v = int(rng.integers(-(1 << 52), 1 << 52)) << int(rng.integers(0, 20))
        f = Fraction(v, 1 << 48)
        d = float(f)
        if Fraction(d) != f:
            continue
        assert orc.fix48_to_f16_bits(v) == int(np.float64(d).astype(np.float16).view(np.uint16))


def test_fix48_rounding_ties_and_overflow(orc):
    # exact midpoints between consecutive fp16 values round to the even one
    for hb in (0x0001, 0x03FF, 0x0400, 0x3C00, 0x3C01, 0x5000, 0x7BFE):
        lo = Fraction(float(np.uint16(hb).view(np.float16)))
        hi = Fraction(float(np.uint16(hb + 1).view(np.float16)))
        mid = (lo + hi) / 2
        v = mid * (1 << 48)
        assert v.denominator == 1
        want = hb if hb % 2 == 0 else hb + 1
        assert orc.fix48_to_f16_bits(int(v)) == want
        assert orc.fix48_to_f16_bits(int(v) + 1) == hb + 1
        assert orc.fix48_to_f16_bits(int(v) - 1) == hb
        assert orc.fix48_to_f16_bits(-int(v) - 1) == (hb + 1) | 0x8000
    assert orc.fix48_to_f16_bits(65520 << 48) == 0x7C00
    assert orc.fix48_to_f16_bits((65520 << 48) - 1) == 0x7BFF
    assert orc.fix48_to_f16_bits(0) == 0
    assert orc.fix48_to_f16_bits(1 << 23) == 0  # 2^-25 is the tie between 0 and 2^-24: even -> 0
    assert orc.fix48_to_f16_bits((1 << 23) + 1) == 1
