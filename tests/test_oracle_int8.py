"""Pins the oracle's INT8 arithmetic.

Reference subset (symmetric int8, zero point 0, round half away from zero):
the known answers of crates/dragonwing-cpu/src/ops.rs:1147-1307 and
crates/dragonwing-core/src/quantization.rs:372-524, and the quantizer's
weight rounding (crates/dragonwing-onnx/src/quantize.rs:520-540).

ONNX extension (QLinearConv / QuantizeLinear / DequantizeLinear /
QLinearAdd / quantized SiLU table — not in the reference): hand-computed
fixtures with exact .5 ties and saturation (tests/golden/qlinear_cases.json),
and an independent numpy evaluation of the ONNX definitions (int64 sums,
np.rint is round-half-even).  Rounding half away instead of half even, or
forgetting the zero point on padded taps, fails these.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_conv2d_i8_all_ones():  # ops.rs:1147-1173
    y = oracle.conv2d_i8_nhwc(np.ones((1, 5, 5, 1), np.int8), np.ones((3, 3, 1, 1), np.int8))
    assert y.shape == (1, 3, 3, 1) and np.all(y == 9)


def test_add_i8():  # ops.rs:1175-1205
    a = np.array([10, 20, 30, 40, 50], np.int8)
    b = np.array([5, 10, 15, 20, 25], np.int8)
    np.testing.assert_array_equal(oracle.add_i8(a, b, 1.0, 1.0), [15, 30, 45, 60, 75])
    c = np.full(3, 100, np.int8)
    np.testing.assert_array_equal(oracle.add_i8(c, c, 0.5, 0.5), [100, 100, 100])


def test_relu_i8():  # ops.rs:1207-1231
    np.testing.assert_array_equal(oracle.relu_i8(np.array([-50, -10, 0, 10, 50], np.int8)), [0, 0, 0, 10, 50])
    x = np.arange(-128, 127).astype(np.int8)
    np.testing.assert_array_equal(oracle.relu_i8(x), np.maximum(x, 0))


def test_requantize():  # ops.rs:1233-1246, quantization.rs requantize_i32_basic
    np.testing.assert_array_equal(
        oracle.requantize_i32_to_i8(np.array([1000, 2000, -1000, -2000, 0], np.int32), 0.1),
        [100, 127, -100, -128, 0])
    np.testing.assert_array_equal(
        oracle.requantize_i32_to_i8(np.array([0, 1000, 5000, -2000, -5000], np.int32), 0.01),
        [0, 10, 50, -20, -50])


def test_requantize_rounds_half_away():
    # f32::round: 2.5 -> 3, -2.5 -> -3, 0.5 -> 1 (ties away from zero).
    np.testing.assert_array_equal(oracle.requantize_i32_to_i8(np.array([5, -5, 1, 3], np.int32), 0.5),
                                  [3, -3, 1, 2])


def test_quantize_dequantize():  # ops.rs:1263-1307
    np.testing.assert_array_equal(
        oracle.quantize_f32_to_i8(np.array([0.0, 5.0, -5.0, 200.0, -200.0], np.float32), 1.0),
        [0, 5, -5, 127, -128])
    np.testing.assert_allclose(oracle.dequantize_i8_to_f32(np.array([0, 10, -10, 127, -128], np.int8), 0.5),
                               [0, 5, -5, 63.5, -64])
    orig = np.array([0.0, 1.5, -2.3, 5.0, -10.0], np.float32)
    back = oracle.dequantize_i8_to_f32(oracle.quantize_f32_to_i8(orig, 0.1), 0.1)
    assert np.all(np.abs(back - orig) < 0.1)


def test_scale_from_range():  # quantization.rs quant_scale_from_range
    assert abs(oracle.scale_from_range(-1.27, 1.27) - 0.01) < 1e-6
    assert abs(oracle.scale_from_range(-0.5, 2.0) - 2.0 / 127.0) < 1e-6
    assert oracle.scale_from_range(0.0, 0.0) == 1.0


def test_weight_quantization():  # quantization.rs per_channel_* and quantize.rs:520-540
    q, s = oracle.quantize_weights_per_channel(
        np.array([[1.27, 0.635, 0.0, -0.635], [2.54, 1.27, 0.0, -1.27]], np.float32))
    np.testing.assert_allclose(s, [1.27 / 127, 2.54 / 127], rtol=1e-6)
    np.testing.assert_array_equal(q[0], [127, 64, 0, -64])
    q2, _ = oracle.quantize_weights_per_channel(np.array([[0.5, 1.0, -0.5, -1.27]], np.float32))
    assert q2[0, 3] == -127


def _np_qlinearconv(x, w, bias, stride, pad, xs, xz, ws, ys, yz):
    """ONNX QLinearConv evaluated independently: pad with x_zp, int64 sums,
    M in f32, np.rint (half to even)."""
    n, h, wd, ci = x.shape
    kh, kw, _, co = w.shape
    ho, wo = oracle.out_hw(h, wd, kh, kw, stride[0], stride[1], pad[0], pad[1])
    xp = np.full((n, h + 2 * pad[0], wd + 2 * pad[1], ci), xz, np.int64)
    xp[:, pad[0]:pad[0] + h, pad[1]:pad[1] + wd] = x
    xp -= xz
    acc = np.zeros((n, ho, wo, co), np.int64)
    for i in range(kh):
        for j in range(kw):
            patch = xp[:, i:i + stride[0] * ho:stride[0], j:j + stride[1] * wo:stride[1], :]
            acc += patch @ w[i, j].astype(np.int64)
    if bias is not None:
        acc += bias
    M = (np.float32(xs) * ws.astype(np.float32)) / np.float32(ys)
    v = acc.astype(np.int32).astype(np.float32) * M
    return np.clip(np.rint(v) + yz, 0, 255).astype(np.uint8)


@pytest.mark.parametrize("geom", [(2, 9, 7, 16, 8, 3, 2, 1), (1, 6, 6, 32, 12, 3, 1, 1),
                                  (1, 5, 8, 16, 4, 1, 1, 0), (3, 4, 4, 48, 20, 3, 2, 1)])
@pytest.mark.parametrize("xz", [128, 0, 37])
def test_qlinearconv_vs_numpy_definition(geom, xz):
    n, h, w, ci, co, k, s, p = geom
    rng = np.random.default_rng(h * 31 + xz)
    x = rng.integers(0, 256, (n, h, w, ci)).astype(np.uint8)
    wt = rng.integers(-127, 128, (k, k, ci, co)).astype(np.int8)
    bias = rng.integers(-4096, 4097, co).astype(np.int32)
    ws = np.exp(rng.uniform(np.log(1e-3), np.log(1e-2), co)).astype(np.float32)
    got = oracle.qlinearconv_u8s8(x, wt, bias, (s, s), (p, p), 0.02, xz, ws, 0.05, 128)
    exp = _np_qlinearconv(x, wt, bias, (s, s), (p, p), 0.02, xz, ws, 0.05, 128)
    np.testing.assert_array_equal(got, exp)


def test_qlinear_golden_fixtures():
    cases = json.loads((GOLDEN / "qlinear_cases.json").read_text())
    for c in cases["qlinearconv"]:
        x = np.array(c["x"], np.uint8).reshape(c["x_shape"])
        w = np.array(c["w"], np.int8).reshape(c["w_shape"])
        bias = np.array(c["bias"], np.int32)
        got = oracle.qlinearconv_u8s8(x, w, bias, c["stride"], c["pad"], c["x_scale"], c["x_zp"],
                                      np.array(c["w_scales"], np.float32), c["y_scale"], c["y_zp"])
        np.testing.assert_array_equal(got.ravel(), c["y"], err_msg=c["name"])
    for c in cases["quantize_linear"]:
        xh = np.array(c["x_f16_bits"], np.uint16)
        np.testing.assert_array_equal(oracle.quantize_linear_f16_u8(xh, c["scale"], c["zp"]), c["y"],
                                      err_msg=c["name"])
    for c in cases["qlinear_add"]:
        got = oracle.qlinear_add_u8(np.array(c["a"], np.uint8), np.array(c["b"], np.uint8), c["sa"], c["za"],
                                    c["sb"], c["zb"], c["sy"], c["zy"])
        np.testing.assert_array_equal(got, c["y"], err_msg=c["name"])


def test_dequantize_linear_and_silu_lut():
    q = np.arange(256, dtype=np.uint8)
    d = oracle.dequantize_linear_u8_f16(q, 0.05, 128)
    np.testing.assert_array_equal(d, ((q.astype(np.float32) - 128) * np.float32(0.05)).astype(np.float16).view(np.uint16))
    lut = oracle.silu_lut_u8(0.05, 128, 0.04, 128)
    v = (q.astype(np.float32) - np.float32(128)) * np.float32(0.05)
    silu = v * (np.float32(1) / (np.float32(1) + np.exp(-v)))
    exp = np.clip(np.rint(silu / np.float32(0.04)) + 128, 0, 255).astype(np.uint8)
    # expf may differ from numpy's exp in the last ulp; allow no more than one
    # table entry to differ by one level.
    diff = np.abs(lut.astype(int) - exp.astype(int))
    assert diff.max() <= 1 and (diff > 0).sum() <= 1
    assert lut[128] == 128  # silu(0) = 0 maps to the zero point
    np.testing.assert_array_equal(oracle.lut_u8(q, lut), lut)
