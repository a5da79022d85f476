"""Pins the oracle's glue and elementwise functions: the reference's own
known-answer tests (crates/dragonwing-cpu/src/ops.rs), closed forms
evaluated independently in numpy, and identities chosen so that plausible
mistakes (a wrong rounding direction, a dropped pad, a swapped operand)
fail."""
import numpy as np
import pytest

import oracle


def test_maxpool_known_answer():  # ops.rs:714-738 maxpool2d_basic
    x = np.arange(16, dtype=np.float32).reshape(1, 4, 4, 1)
    np.testing.assert_array_equal(oracle.maxpool2d_f32(x, (2, 2), (2, 2)).ravel(), [5, 7, 13, 15])


def _padded_max_numpy(x, k, s, pads):
    pt, pl, pb, pr = pads
    xp = np.pad(x.astype(np.float64), ((0, 0), (pt, pb), (pl, pr), (0, 0)), constant_values=-np.inf)
    n, h, w, c = xp.shape
    ho, wo = (h - k) // s + 1, (w - k) // s + 1
    y = np.empty((n, ho, wo, c))
    for i in range(ho):
        for j in range(wo):
            y[:, i, j, :] = xp[:, i * s:i * s + k, j * s:j * s + k, :].max(axis=(1, 2))
    return y


@pytest.mark.parametrize("k,s,p", [(5, 1, 2), (3, 2, 1), (2, 2, 0)])
def test_padded_maxpool_matches_definition(k, s, p):
    # ONNX MaxPool: padded positions never win (all-negative input: a zero
    # pad would leak into the border outputs).
    x = -np.abs(np.random.default_rng(k).normal(size=(2, 9, 7, 3))).astype(np.float32) - 0.5
    y = oracle.maxpool2d_padded(x, (k, k), (s, s), (p, p, p, p))
    np.testing.assert_array_equal(y, _padded_max_numpy(x, k, s, (p, p, p, p)).astype(np.float32))
    assert (y < 0).all()


def test_sppf_cascade_identity():
    # A 5x5 stride-1 pad-2 pool applied twice is one 9x9 pool, thrice a 13x13
    # pool (the SPPF cascade the runtime fuses).
    x = np.random.default_rng(1).normal(size=(1, 11, 13, 4)).astype(np.float32)
    p1 = oracle.maxpool2d_padded(x, (5, 5), (1, 1), (2, 2, 2, 2))
    p2 = oracle.maxpool2d_padded(p1, (5, 5), (1, 1), (2, 2, 2, 2))
    p3 = oracle.maxpool2d_padded(p2, (5, 5), (1, 1), (2, 2, 2, 2))
    np.testing.assert_array_equal(p2, oracle.maxpool2d_padded(x, (9, 9), (1, 1), (4, 4, 4, 4)))
    np.testing.assert_array_equal(p3, oracle.maxpool2d_padded(x, (13, 13), (1, 1), (6, 6, 6, 6)))


def test_resize_nearest_known_answer():  # ops.rs:964-984 resize_f32_nearest_2x
    x = np.array([1, 2, 3, 4], np.float32).reshape(1, 2, 2, 1)
    np.testing.assert_array_equal(oracle.resize_nearest(x, 4, 4).ravel(),
                                  [1, 1, 2, 2, 1, 1, 2, 2, 3, 3, 4, 4, 3, 3, 4, 4])


@pytest.mark.parametrize("hw", [((3, 5), (5, 8)), ((7, 4), (3, 9)), ((20, 20), (40, 40))])
def test_resize_nearest_index_rule(hw):
    # ih = clamp(round((oh + 0.5) * h_in/h_out - 0.5)) with f32 arithmetic and
    # round half away from zero (Rust f32::round), ops.rs:2336-2342.
    (h, w), (ho, wo) = hw
    x = np.arange(h * w * 2, dtype=np.float32).reshape(1, h, w, 2)

    def idx(o, n_in, n_out):
        v = np.float32(np.float32(np.float32(o) + np.float32(0.5)) * np.float32(np.float32(n_in) / np.float32(n_out)))
        v = np.float32(v - np.float32(0.5))
        r = np.floor(np.abs(v) + 0.5) * np.sign(v)
        return int(min(max(r, 0.0), n_in - 1))

    exp = np.empty((1, ho, wo, 2), np.float32)
    for i in range(ho):
        for j in range(wo):
            exp[0, i, j] = x[0, idx(i, h, ho), idx(j, w, wo)]
    np.testing.assert_array_equal(oracle.resize_nearest(x, ho, wo), exp)


def test_concat_known_answer():  # ops.rs:919-944 concat_f32_channels
    a = np.arange(1, 9, dtype=np.float32).reshape(1, 2, 2, 2)
    b = (np.arange(1, 9, dtype=np.float32) * 10).reshape(1, 2, 2, 2)
    np.testing.assert_array_equal(oracle.concat_channels([a, b]).ravel(),
                                  [1, 2, 10, 20, 3, 4, 30, 40, 5, 6, 50, 60, 7, 8, 70, 80])


def test_split_known_answer_and_inverse():  # ops.rs:1008-1029 split_f32_channels
    x = np.arange(16, dtype=np.float32).reshape(1, 2, 2, 4)
    o1, o2 = oracle.split_channels(x, [2, 2])
    assert o1.ravel()[:2].tolist() == [0, 1] and o2.ravel()[:2].tolist() == [2, 3]
    y = np.random.default_rng(2).integers(0, 255, (2, 3, 5, 7)).astype(np.uint8)
    np.testing.assert_array_equal(oracle.concat_channels(oracle.split_channels(y, [3, 1, 3])), y)


def test_sigmoid_known_answer():  # ops.rs:860-874 sigmoid_f32_basic (+-0.01)
    y = oracle.sigmoid_f32(np.array([-2, -1, 0, 1, 2], np.float32))
    assert np.all(np.abs(y - np.array([0.119, 0.269, 0.5, 0.731, 0.881])) < 0.01)
    # and the closed form within a few ulps (expf is the host libm's)
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    ref = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    assert np.max(np.abs(oracle.sigmoid_f32(x) - ref)) <= 4 * np.finfo(np.float32).eps


def test_float_elementwise_closed_forms():
    rng = np.random.default_rng(3)
    a = rng.normal(size=1000).astype(np.float32)
    b = rng.normal(size=1000).astype(np.float32)
    np.testing.assert_array_equal(oracle.add_f32(a, b), a + b)
    np.testing.assert_array_equal(oracle.mul_f32(a, b), a * b)
    # relu_f32_scalar (ops.rs:208-220): x > 0 ? x : +0, NaN propagates
    r = oracle.relu_f32(np.array([-1.0, -0.0, 0.0, 2.0, np.nan], np.float32))
    assert r[:4].tolist() == [0.0, 0.0, 0.0, 2.0] and np.isnan(r[4])
    assert not np.signbit(r[1])
    # f16 ops: widen, operate in f32, round once to f16 (normal range, where
    # the reference decode is IEEE)
    ha = oracle.f16_from_f32(a)
    hb = oracle.f16_from_f32(b)
    fa, fb = ha.view(np.float16).astype(np.float32), hb.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(oracle.add_fp16(ha, hb), (fa + fb).astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(oracle.mul_fp16(ha, hb), (fa * fb).astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(oracle.relu_fp16(ha), np.maximum(fa, 0).astype(np.float16).view(np.uint16))


def test_quantize_linear_ties_and_saturation():
    # y = clamp(rint(x / s) + zp): ties to even (2.5 -> 2, 3.5 -> 4), saturation
    s = 0.5
    x = np.array([1.25, 1.75, -1.25, 1000.0, -1000.0, 0.0], np.float32)
    got = oracle.quantize_linear_f16_u8(oracle.f16_from_f32(x), s, 128)
    assert got.tolist() == [130, 132, 126, 255, 0, 128]
    v = np.random.default_rng(4).normal(0, 3, 5000).astype(np.float32)
    h = oracle.f16_from_f32(v)
    exp = np.clip(np.rint(h.view(np.float16).astype(np.float32) / np.float32(0.037)) + 100, 0, 255)
    np.testing.assert_array_equal(oracle.quantize_linear_f16_u8(h, 0.037, 100), exp.astype(np.uint8))


def test_dequantize_linear_and_qlinear_add_closed_forms():
    q = np.arange(256, dtype=np.uint8)
    exp = ((q.astype(np.int32) - 131).astype(np.float32) * np.float32(0.0213)).astype(np.float16)
    np.testing.assert_array_equal(oracle.dequantize_linear_u8_f16(q, 0.0213, 131), exp.view(np.uint16))
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, 4000).astype(np.uint8)
    b = rng.integers(0, 256, 4000).astype(np.uint8)
    sa, sb, sy = np.float32(0.031), np.float32(0.017), np.float32(0.043)
    f = (a.astype(np.int32) - 120).astype(np.float32) * (sa / sy) + (b.astype(np.int32) - 135).astype(np.float32) * (sb / sy)
    exp = np.clip(np.rint(f) + 128, 0, 255).astype(np.uint8)
    np.testing.assert_array_equal(oracle.qlinear_add_u8(a, b, sa, 120, sb, 135, sy, 128), exp)
    lut = rng.integers(0, 256, 256).astype(np.uint8)
    np.testing.assert_array_equal(oracle.lut_u8(a, lut), lut[a])
