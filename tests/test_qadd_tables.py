"""The shortcut's QLinearAdd in the chained-pair and C2f kernels from two
tables of rounded products (IgemmArgs::rtab, built by the runtime for a
table epilogue with a residual): entry q of the first is f32((lut[q] - za) *
ra), entry b of the second f32((b - zb) * rb).  The kernels add two entries
(the reference's sum of its two rounded products), round to the nearest even
integer by adding 1.5 * 2^23, and clamp the biased value to the zero point's
0..255 range with one med3.  Restated here in float32 numpy exactly as the
kernels compute it, against the oracle's QLinearAdd (oracle/dw_oracle.cpp,
dwo_qlinear_add_u8) on every pair of operand bytes."""
import numpy as np
import pytest

import oracle

C = np.float32(12582912.0)  # 1.5 * 2^23


def tables(lut, sa, za, sb, zb, sy):
    ra = np.float32(sa) / np.float32(sy)
    rb = np.float32(sb) / np.float32(sy)
    q = np.arange(256, dtype=np.int32)
    ta = (lut.astype(np.int32) - za).astype(np.float32) * ra
    tb = (q - zb).astype(np.float32) * rb
    return ta.astype(np.float32), tb.astype(np.float32)


def kernel_add(ta, tb, qt, b, zy, round_fn=None):
    s = ta[qt] + tb[b]
    if round_fn is not None:  # a planted mistake: another rounding of the sum
        return np.clip(round_fn(s) + zy, 0, 255).astype(np.uint8)
    lo = np.float32(C - np.float32(zy))
    t = np.minimum(np.maximum(s + C, lo), lo + np.float32(255.0))
    return (t.view(np.int32) - (0x4B400000 - zy)).astype(np.uint8)


CASES = [
    # (sa, za, sb, zb, sy, zy): the graph's zero points (128), others, and
    # scale ratios 1 and 1/2, whose sums land on .5 exactly (ties)
    (0.05, 128, 0.05, 128, 0.05, 128),
    (0.04, 128, 0.02, 128, 0.04, 128),
    (0.031, 128, 0.017, 128, 0.023, 128),
    (0.2, 0, 0.01, 255, 0.07, 77),
    (0.011, 200, 0.13, 3, 0.05, 0),
    (0.0042, 128, 0.0091, 128, 0.0063, 255),
]


@pytest.mark.parametrize("sa,za,sb,zb,sy,zy", CASES)
@pytest.mark.parametrize("table", ["identity", "silu"])
def test_qadd_tables_match_oracle(sa, za, sb, zb, sy, zy, table):
    lut = np.arange(256, dtype=np.uint8) if table == "identity" else oracle.silu_lut_u8(sa * 1.3, 128, sa, za)
    ta, tb = tables(lut, sa, za, sb, zb, sy)
    assert np.abs(ta).max() + np.abs(tb).max() < 2.0 ** 21  # the runtime's condition for the tables
    qt, b = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    got = kernel_add(ta, tb, qt, b, zy)
    ref = oracle.qlinear_add_u8(lut[qt], b.astype(np.uint8), sa, za, sb, zb, sy, zy)
    np.testing.assert_array_equal(got, ref)
    assert len(np.unique(ref)) > 32


def test_qadd_tables_ties_pin_the_rounding():
    # ratio 1/2: half of the sums are ties; rounding them away from zero
    # (not to even) fails against the oracle, the kernels' add does not
    sa, za, sb, zb, sy, zy = 0.04, 128, 0.02, 128, 0.04, 128
    lut = np.arange(256, dtype=np.uint8)
    ta, tb = tables(lut, sa, za, sb, zb, sy)
    qt, b = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    ref = oracle.qlinear_add_u8(lut[qt], b.astype(np.uint8), sa, za, sb, zb, sy, zy)
    np.testing.assert_array_equal(kernel_add(ta, tb, qt, b, zy), ref)
    away = kernel_add(ta, tb, qt, b, zy, round_fn=lambda s: np.sign(s) * np.floor(np.abs(s) + 0.5))
    assert np.any(away != ref)
