"""Pins the oracle's activations and their rounding points:

* ``sigmoid_fp16`` (ops.rs:1881-1888): decode with F16::to_f32, one f32
  sigmoid ``1 / (1 + exp(-x))``, one F16 rounding.  Checked on all 65,536
  inputs against the sigmoid evaluated in f64 and rounded to binary16 by
  numpy: wherever the f32 evaluation error (a few f32 ulps) cannot move the
  value across an f16 rounding boundary the oracle must agree exactly, and
  elsewhere it must be one of the two neighbours.  The reference's own
  tolerance test (ops.rs:860-874) is included.
* ``silu_fp16`` = Sigmoid then Mul, each rounded to f16 (runtime.rs:1641-1734):
  the product of two f16 values is exact in f64, so the Mul is the RNE
  rounding of an exact product of the two *decoded* operands.  The decode is
  the reference's (subnormals at half value, dtype.rs:236-248), which matters
  here because the sigmoid of x below about -9.7 is an f16 subnormal.
* ``clip`` (runtime.rs:1004-1042): Rust ``f32::clamp`` (NaN passes, -0.0 kept)
  on f32, and the F16 round trip (decode, clamp, encode) on f16, from a hand
  table.
* ``softmax_f32`` / ``softmax_f16`` (ops.rs:1609-1638, runtime.rs:1311-1322):
  against the f64 closed form with the same ambiguity-band rule, the
  reference's known answer (ops.rs:765-777), overflow-safe rows (the max
  subtraction) and NaN / infinity rows from the f32::max fold.

Each check is built so that a plausible mistake fails it; the mistakes are
planted in copies of the oracle's arithmetic below, on the CPU.
"""
import numpy as np

import oracle

ALL = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def ref_decode(h):
    """F16::to_f32_soft, restated from IEEE binary16 with the reference's one
    deviation: subnormals decode to half their IEEE value."""
    h = np.asarray(h, np.uint16)
    v = h.view(np.float16).astype(np.float64)
    sub = ((h & 0x7C00) == 0) & ((h & 0x3FF) != 0)
    with np.errstate(invalid="ignore"):
        return np.where(sub, v * 0.5, v)


def rne16(v64):
    """IEEE binary16 round-to-nearest-even of f64 values (numpy's direct
    double-to-half conversion), as bit patterns."""
    with np.errstate(over="ignore"):
        return np.asarray(v64, np.float64).astype(np.float16).view(np.uint16)


def banded(v64, rel):
    """(lo, hi) f16 encodings of v·(1∓rel): equal where an evaluation with
    relative error below rel cannot change the rounded result."""
    lo = rne16(v64 * (1.0 - rel))
    hi = rne16(v64 * (1.0 + rel))
    neg = v64 < 0
    return np.where(neg, hi, lo), np.where(neg, lo, hi)


def check_banded(got, v64, rel, min_exact_frac=0.99):
    lo, hi = banded(v64, rel)
    sure = lo == hi
    np.testing.assert_array_equal(got[sure], lo[sure])
    unsure = ~sure
    assert np.all((got[unsure] == lo[unsure]) | (got[unsure] == hi[unsure]))
    assert sure.mean() >= min_exact_frac
    return sure


def sigmoid64(x):
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-x))


# --- sigmoid_fp16 ------------------------------------------------------------

FINITE = ~(((ALL & 0x7C00) == 0x7C00))


def test_sigmoid_fp16_all_inputs():
    got = oracle.sigmoid_fp16(ALL)
    x = ref_decode(ALL)
    # f32 evaluation: expf (<= 1 ulp), one add, one divide: < 4 f32 ulps.
    check_banded(got[FINITE], sigmoid64(x[FINITE]), 4 * 2.0**-24)
    assert got[0x7C00] == 0x3C00  # sigmoid(+inf) = 1
    assert got[0xFC00] == 0x0000  # sigmoid(-inf) = +0
    nan = ~FINITE & ((ALL & 0x3FF) != 0)
    assert np.all(np.isnan(oracle.f16_to_f32(got[nan])))


def test_sigmoid_reference_known_answer():  # ops.rs:860-874 sigmoid_f32_basic
    x = np.array([-2.0, -1.0, 0.0, 1.0, 2.0], np.float32)
    y = oracle.sigmoid_f32(x)
    assert np.all(np.abs(y - np.array([0.119, 0.269, 0.5, 0.731, 0.881])) < 0.01)
    assert y[2] == 0.5
    h = oracle.f16_from_f32(x)
    assert oracle.f16_to_f32(oracle.sigmoid_fp16(h))[2] == 0.5


def test_sigmoid_f32_closed_form():
    x = np.random.default_rng(7).uniform(-30, 30, 200_000).astype(np.float32)
    y = oracle.sigmoid_f32(x).astype(np.float64)
    s = sigmoid64(x.astype(np.float64))
    assert np.all(np.abs(y - s) <= 4 * 2.0**-24 * s + 1e-45)


def test_sigmoid_fp16_planted_mistakes_fail():
    x = ref_decode(ALL[FINITE])
    s = sigmoid64(x)
    lo, hi = banded(s, 4 * 2.0**-24)
    sure = lo == hi
    # exp(x) in place of exp(-x)
    wrong_sign = rne16(1.0 / (1.0 + np.exp(np.minimum(x, 80))))
    assert np.any(wrong_sign[sure] != lo[sure])
    # the f32 result truncated to f16 instead of rounded
    s32 = s.astype(np.float32)
    trunc = (s32.view(np.uint32) >> 13).astype(np.uint16)
    norm = s32 >= 2.0**-14
    assert np.any(trunc[sure & norm] != lo[sure & norm])
    # the whole sigmoid in f16 arithmetic (exp, add and divide each rounded)
    with np.errstate(over="ignore"):
        e16 = np.exp(-x.astype(np.float16).astype(np.float64)).astype(np.float16)
    d16 = (np.float16(1) + e16).astype(np.float16)
    in_f16 = (np.float16(1) / d16).astype(np.float16).view(np.uint16)
    assert np.any(in_f16[sure] != lo[sure])


# --- silu_fp16 ---------------------------------------------------------------

def test_silu_fp16_is_rounded_product_of_rounded_sigmoid():
    got = oracle.silu_fp16(ALL)
    sig = oracle.sigmoid_fp16(ALL)
    f = FINITE
    # exact product of the two decoded f16 operands, one RNE rounding
    np.testing.assert_array_equal(got[f], rne16(ref_decode(ALL[f]) * ref_decode(sig[f])))
    # the rounding of the sigmoid before the Mul is visible: multiplying by the
    # unrounded sigmoid gives different bits on a large share of inputs
    direct = rne16(ref_decode(ALL[f]) * sigmoid64(ref_decode(ALL[f])))
    assert np.mean(direct != got[f]) > 0.01
    # the reference decode matters where the sigmoid is an f16 subnormal
    ieee = rne16(ALL[f].view(np.float16).astype(np.float64) * sig[f].view(np.float16).astype(np.float64))
    sub_sig = ((sig[f] & 0x7C00) == 0) & ((sig[f] & 0x3FF) != 0)
    assert sub_sig.sum() > 100
    assert np.any(ieee[sub_sig] != got[f][sub_sig])


# --- clip --------------------------------------------------------------------

def test_clip_f32_table():
    nan = np.float32("nan")
    x = np.array([nan, -np.inf, -1.0, -0.0, 0.0, 0.05, 3.0, 6.0, 6.5, np.inf], np.float32)
    y = oracle.clip(x, 0.0, 6.0)
    want = np.array([nan, 0.0, 0.0, -0.0, 0.0, 0.05, 3.0, 6.0, 6.0, 6.0], np.float32)
    assert np.isnan(y[0])
    np.testing.assert_array_equal(y[1:].view(np.uint32), want[1:].view(np.uint32))  # -0.0 kept


def test_clip_f16_table():
    # lo = 0.1 is not an f16 value: a clamped output is F16::from_f32(0.1f32).
    rows = [
        (0x0000, 0x2E66),  # +0 below 0.1 -> F16(0.1) = 0x2E66 (0.0999755859375)
        (0x3C00, 0x3C00),  # 1.0 inside
        (0x4600, 0x4500),  # 6.0 above hi = 5.0
        (0x7C00, 0x4500),  # +inf -> hi
        (0xFC00, 0x2E66),  # -inf -> lo
        # NaN passes; decode gives 0x7FC00000 and the encoder's payload is
        # min(mant >> 13, 0x1FF) (dtype.rs:176), so 0x7E00 comes back as 0x7FFF
        (0x7E00, 0x7FFF),
    ]
    x = np.array([r[0] for r in rows], np.uint16)
    y = oracle.clip(x, 0.1, 5.0)
    np.testing.assert_array_equal(y, [r[1] for r in rows])
    # A subnormal inside [lo, hi] is not returned unchanged: the decode halves
    # it and the encode keeps the halved value (0x0002 -> 0x0001).
    y = oracle.clip(np.array([0x0002, 0x8004, 0x03FF], np.uint16), -1.0, 1.0)
    np.testing.assert_array_equal(y, [0x0001, 0x8002, 0x0200])
    # -0.0 inside the range keeps its sign
    assert oracle.clip(np.array([0x8000], np.uint16), -1.0, 1.0)[0] == 0x8000


def test_clip_f16_all_inputs():
    lo, hi = -2.5, 3.3
    got = oracle.clip(ALL, lo, hi)
    x = ref_decode(ALL)
    lo32, hi32 = np.float64(np.float32(lo)), np.float64(np.float32(hi))
    c = np.where(x < lo32, lo32, np.where(x > hi32, hi32, x))
    want = rne16(c)
    real = ~np.isnan(x)
    np.testing.assert_array_equal(got[real], want[real])
    assert np.all(np.isnan(oracle.f16_to_f32(got[~real])))


# --- softmax -------------------------------------------------------------------

def softmax64(x):
    x = np.asarray(x, np.float64)
    m = np.max(np.where(np.isnan(x), -np.inf, x), axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = np.exp(x - m)
        return e / e.sum(axis=-1, keepdims=True)


def test_softmax_reference_known_answer():  # ops.rs:765-777 softmax_basic
    y = oracle.softmax_f32(np.array([[1.0, 2.0, 3.0]], np.float32))[0]
    assert abs(float(y.sum()) - 1.0) < 1e-5 and y[0] < y[1] < y[2] and np.all(y > 0)


def test_softmax_f32_closed_form():
    x = np.random.default_rng(3).normal(0, 4, size=(4000, 16)).astype(np.float32)
    y = oracle.softmax_f32(x).astype(np.float64)
    p = softmax64(x)
    # expf per term, a sum of 16 and one multiply by the reciprocal
    assert np.all(np.abs(y - p) <= 24 * 2.0**-24 * p + 1e-44)


def test_softmax_f16_closed_form():
    rng = np.random.default_rng(11)
    n = 16  # the DFL bin count
    xh = oracle.f16_from_f32(rng.normal(0, 3, size=(8000, n)).astype(np.float32))
    got = oracle.softmax_f16(xh)
    p = softmax64(ref_decode(xh))
    check_banded(got.ravel(), p.ravel(), (n + 8) * 2.0**-24)


def test_softmax_f16_special_rows():
    big = oracle.f16_from_f32(np.linspace(90, 100, 16).astype(np.float32))  # exp(100) overflows f32
    nan_row = big.copy()
    nan_row[3] = 0x7E00
    inf_row = oracle.f16_from_f32(np.zeros(16, np.float32))
    inf_row[5] = 0x7C00
    neg_inf = oracle.f16_from_f32(np.zeros(16, np.float32))
    neg_inf[:8] = 0xFC00
    rows = np.stack([big, nan_row, inf_row, neg_inf])
    got = oracle.softmax_f16(rows)
    f = oracle.f16_to_f32(got)
    # the max subtraction keeps the large row finite and summing to ~1
    np.testing.assert_array_equal(got[0], rne16(softmax64(ref_decode(big))))
    assert abs(float(f[0].sum()) - 1.0) < 1e-2
    # NaN loses the f32::max fold, then exp(NaN) poisons the sum: all NaN
    assert np.all(np.isnan(f[1]))
    # +inf is the max: inf - inf = NaN, and the whole row is NaN
    assert np.all(np.isnan(f[2]))
    # -inf entries weigh exactly 0, the rest share equally (1/8 exactly)
    np.testing.assert_array_equal(f[3][:8], 0.0)
    np.testing.assert_array_equal(f[3][8:], 0.125)


def test_softmax_f16_planted_mistakes_fail():
    rng = np.random.default_rng(12)
    xh = oracle.f16_from_f32(rng.normal(0, 3, size=(2000, 16)).astype(np.float32))
    p = softmax64(ref_decode(xh)).ravel()
    lo, hi = banded(p, 24 * 2.0**-24)
    sure = lo == hi
    # softmax with exp and the sum carried in f16
    x16 = ref_decode(xh).astype(np.float16)
    e16 = np.exp((x16 - x16.max(axis=1, keepdims=True)).astype(np.float64)).astype(np.float16)
    s16 = np.zeros((x16.shape[0], 1), np.float16)
    for j in range(16):
        s16 = (s16 + e16[:, j:j + 1]).astype(np.float16)
    in_f16 = (e16 / s16).astype(np.float16).view(np.uint16).ravel()
    assert np.any(in_f16[sure] != lo[sure])
    # no max subtraction: exp overflows f32 on the large row
    big = np.linspace(90, 100, 16).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(big)
        naive = e / e.sum()
    assert np.any(np.isnan(naive)) and not np.any(np.isnan(oracle.softmax_f32(big[None])))
