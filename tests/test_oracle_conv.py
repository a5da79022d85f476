"""Pins the oracle's convolutions (conv2d_f32_nhwc(_mt), conv2d_fp16_nhwc_mt,
depthwise_*_mt; crates/dragonwing-cpu/src/ops.rs) and the CpuGraphRuntime
bias pass (crates/dragonwing-onnx/src/runtime.rs:1445-1498).

Checks: the reference's known answers (ops.rs:652-712, :811-854;
vulkan_runtime.rs:2886-2936), an f64 brute force on small random shapes
(exact up to f32 rounding), exactness of the single-FMA order on inputs
where every partial sum is representable, torch's F.conv2d as an
independent library cross-check, and the depthwise closed form (9/6/4 for
an all-ones 3x3 with padding 1).
"""
import numpy as np
import pytest

import oracle


def brute_f64(x, k, stride, pad):
    n, h, w, ci = x.shape
    kh, kw, _, co = k.shape
    ho, wo = oracle.out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    xp = np.zeros((n, h + 2 * pad[0], w + 2 * pad[1], ci))
    xp[:, pad[0]:pad[0] + h, pad[1]:pad[1] + w] = x
    y = np.zeros((n, ho, wo, co))
    for i in range(kh):
        for j in range(kw):
            patch = xp[:, i:i + stride[0] * ho:stride[0], j:j + stride[1] * wo:stride[1], :]
            y += patch.astype(np.float64) @ k[i, j].astype(np.float64)
    return y


def test_identity_1x1():  # ops.rs:652-680
    x = (np.arange(1 * 4 * 4 * 2, dtype=np.float32) * np.float32(0.1)).reshape(1, 4, 4, 2)
    k = np.zeros((1, 1, 2, 2), np.float32)
    k[0, 0, 0, 0] = k[0, 0, 1, 1] = 1.0
    np.testing.assert_array_equal(oracle.conv2d_f32_nhwc(x, k), x)


def test_all_ones_3x3():  # ops.rs:682-712
    y = oracle.conv2d_f32_nhwc(np.ones((1, 5, 5, 1), np.float32), np.ones((3, 3, 1, 1), np.float32))
    assert y.shape == (1, 3, 3, 1) and np.all(y == 9.0)


def test_mt_matches_st_sin_cos():  # ops.rs:811-854 (and bitwise, since the per-output order is fixed)
    x = np.sin(np.arange(14 * 14 * 16, dtype=np.float32) * np.float32(0.01)).reshape(1, 14, 14, 16)
    k = np.cos(np.arange(9 * 16 * 32, dtype=np.float32) * np.float32(0.02)).reshape(3, 3, 16, 32)
    st = oracle.conv2d_f32_nhwc_st(x, k, (1, 1), (1, 1))
    mt = oracle.conv2d_f32_nhwc(x, k, (1, 1), (1, 1), threads=4)
    np.testing.assert_array_equal(st, mt)
    np.testing.assert_allclose(st, brute_f64(x, k, (1, 1), (1, 1)), rtol=1e-4, atol=1e-4)


def test_conv_with_bias_worked_example():  # vulkan_runtime.rs:2886-2936
    x = (np.arange(36, dtype=np.float32) * np.float32(0.1) - np.float32(1.0)).reshape(1, 3, 3, 4)
    w = np.array([0.5, -0.25, 0.1, 0.2, -0.3, 0.4, 0.7, 0.0], np.float32).reshape(1, 1, 4, 2)
    b = np.array([100.0, -50.0], np.float32)
    y = oracle.bias_add_f32(oracle.conv2d_f32_nhwc(x, w), b)
    exp = x.reshape(9, 4).astype(np.float64) @ w.reshape(4, 2).astype(np.float64) + b
    np.testing.assert_allclose(y.reshape(9, 2), exp, atol=1e-4)


@pytest.mark.parametrize("shape", [(2, 7, 9, 5, 6, 3, 1, 1), (1, 8, 8, 16, 8, 3, 2, 1),
                                   (1, 6, 5, 3, 16, 3, 2, 1), (2, 5, 5, 4, 4, 1, 1, 0)])
def test_brute_force_f64(shape):
    n, h, w, ci, co, k, s, p = shape
    rng = np.random.default_rng(7)
    x = rng.uniform(-1, 1, (n, h, w, ci)).astype(np.float32)
    kk = rng.uniform(-1, 1, (k, k, ci, co)).astype(np.float32)
    y = oracle.conv2d_f32_nhwc(x, kk, (s, s), (p, p))
    np.testing.assert_allclose(y, brute_f64(x, kk, (s, s), (p, p)), rtol=1e-5, atol=1e-5)


def test_exact_on_dyadic_inputs():
    # Small-integer inputs/weights: every partial sum is an exact f32, so the
    # oracle must equal the f64 brute force bit for bit (a dropped tap, a
    # wrong pad offset or a transposed kernel cannot hide).
    rng = np.random.default_rng(3)
    x = rng.integers(-8, 9, (2, 9, 7, 6)).astype(np.float32)
    k = rng.integers(-4, 5, (3, 3, 6, 5)).astype(np.float32)
    for s, p in [(1, 1), (2, 1), (2, 0), (1, 0)]:
        np.testing.assert_array_equal(oracle.conv2d_f32_nhwc(x, k, (s, s), (p, p)),
                                      brute_f64(x, k, (s, s), (p, p)).astype(np.float32))


def test_torch_cross_check_cfg1_shape():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = rng.uniform(-1, 1, (1, 56, 56, 64)).astype(np.float32)
    k = rng.uniform(-1, 1, (3, 3, 64, 64)).astype(np.float32)
    y = oracle.conv2d_f32_nhwc(x, k, (1, 1), (1, 1))
    t = torch.nn.functional.conv2d(torch.from_numpy(x.transpose(0, 3, 1, 2)).double(),
                                   torch.from_numpy(k.transpose(3, 2, 0, 1)).double(), padding=1)
    np.testing.assert_allclose(y, t.numpy().transpose(0, 2, 3, 1), rtol=1e-4, atol=1e-4)


def test_fp16_conv_is_f32_conv_of_widened_operands():
    rng = np.random.default_rng(5)
    xh = rng.normal(0, 1, (1, 10, 10, 16)).astype(np.float16).view(np.uint16)
    kh = rng.normal(0, 0.1, (3, 3, 16, 8)).astype(np.float16).view(np.uint16)
    y = oracle.conv2d_fp16_nhwc(xh, kh, (1, 1), (1, 1))
    y32 = oracle.conv2d_f32_nhwc(oracle.f16_to_f32(xh), oracle.f16_to_f32(kh), (1, 1), (1, 1))
    np.testing.assert_array_equal(y, oracle.f16_from_f32(y32))


def test_bias_add_f16_double_rounding():
    # runtime.rs:1483-1498: F16(f32(out) + f32(bias)).
    y = np.array([0x3C00, 0x3C01], np.uint16)  # 1.0, 1.0 + 2^-10
    b = np.array([0x1400, 0x1400], np.uint16)  # 2^-10 (same column twice via 2 pixels)
    out = oracle.bias_add_f16(y.reshape(2, 1), b[:1])
    # 1 + 2^-10 is representable -> 0x3C01; (1+2^-10)+2^-10 = 1+2^-9 -> 0x3C02
    np.testing.assert_array_equal(out.ravel(), [0x3C01, 0x3C02])


def test_depthwise_closed_form():
    x = np.ones((1, 6, 5, 8), np.float32)
    k = np.ones((3, 3, 8), np.float32)
    y = oracle.depthwise_f32(x, k, (1, 1), (1, 1))
    exp = np.full((6, 5), 9.0)
    exp[0, :] = exp[-1, :] = 6.0
    exp[:, 0] = exp[:, -1] = 6.0
    exp[0, 0] = exp[0, -1] = exp[-1, 0] = exp[-1, -1] = 4.0
    for c in range(8):
        np.testing.assert_array_equal(y[0, :, :, c], exp)


def test_depthwise_equals_per_channel_conv():
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (2, 7, 6, 8)).astype(np.float32)
    k = rng.normal(0, 0.1, (3, 3, 8)).astype(np.float32)
    y = oracle.depthwise_f32(x, k, (2, 2), (1, 1))
    for c in range(8):
        yc = oracle.conv2d_f32_nhwc(np.ascontiguousarray(x[..., c:c + 1]),
                                    np.ascontiguousarray(k[:, :, c:c + 1, None]), (2, 2), (1, 1))
        np.testing.assert_array_equal(y[..., c:c + 1], yc)


def test_depthwise_fp16_is_f32_of_widened():
    rng = np.random.default_rng(11)
    xh = rng.normal(0, 1, (1, 8, 8, 16)).astype(np.float16).view(np.uint16)
    kh = rng.normal(0, 0.1, (3, 3, 16)).astype(np.float16).view(np.uint16)
    y = oracle.depthwise_fp16(xh, kh, (1, 1), (1, 1))
    y32 = oracle.depthwise_f32(oracle.f16_to_f32(xh), oracle.f16_to_f32(kh), (1, 1), (1, 1))
    np.testing.assert_array_equal(y, oracle.f16_from_f32(y32))


def test_fold_batchnorm_closed_form():
    rng = np.random.default_rng(2)
    w = rng.normal(0, 1, (4, 3, 3, 3)).astype(np.float32)
    g, beta, mean = (rng.uniform(0.5, 1.5, 4).astype(np.float32), rng.normal(0, .1, 4).astype(np.float32),
                     rng.normal(0, .1, 4).astype(np.float32))
    var = rng.uniform(0.5, 1.5, 4).astype(np.float32)
    w2, b2 = oracle.fold_batchnorm(w, None, g, beta, mean, var, 1e-3)
    sf = g.astype(np.float64) / np.sqrt(var.astype(np.float64) + np.float64(np.float32(1e-3)))
    np.testing.assert_array_equal(w2, (w.astype(np.float64) * sf[:, None, None, None]).astype(np.float32))
    np.testing.assert_array_equal(b2, ((0 - mean.astype(np.float64)) * sf + beta).astype(np.float32))


# --- accumulation order, in exact rationals ----------------------------------
from fractions import Fraction  # noqa: E402


def _round_f32(q: Fraction) -> Fraction:
    """q rounded to the nearest binary32 value, ties to even (subnormals
    included; the magnitudes here never overflow)."""
    if q == 0:
        return Fraction(0)
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    n = m.numerator // m.denominator
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return (n * ulp) if q > 0 else -(n * ulp)


def _conv_exact(x, w, pad, order="kh_kw_ic", fused=True):
    """Direct convolution whose every step is one rounding to f32 of the
    exact value: fma(x, w, acc) when fused, else round(round(x*w) + acc).
    order names the loop nesting of the taps, outermost first."""
    n, h, wd, ci = x.shape
    kh, kw, _, co = w.shape
    ho, wo = h + 2 * pad - kh + 1, wd + 2 * pad - kw + 1
    X = [[[[Fraction(float(v)) for v in px] for px in row] for row in img] for img in x]
    W = [[[[Fraction(float(w[a, b, c, d])) for d in range(co)] for c in range(ci)] for b in range(kw)] for a in range(kh)]
    taps = [(a, b, c) for a in range(kh) for b in range(kw) for c in range(ci)]
    if order == "ic_kh_kw":
        taps.sort(key=lambda t: (t[2], t[0], t[1]))
    y = np.zeros((n, ho, wo, co), np.float32)
    for b_ in range(n):
        for oh in range(ho):
            for ow in range(wo):
                for oc in range(co):
                    acc = Fraction(0)
                    for a, b, c in taps:
                        ih, iw = oh + a - pad, ow + b - pad
                        if not (0 <= ih < h and 0 <= iw < wd):
                            continue  # out-of-image taps are skipped, as ops.rs:1402-1410 does
                        p = X[b_][ih][iw][c] * W[a][b][c][oc]
                        acc = _round_f32(acc + p) if fused else _round_f32(acc + _round_f32(p))
                    y[b_, oh, ow, oc] = np.float32(float(acc))
    return y


def test_conv_accumulation_order_pinned_in_exact_rationals():
    # conv2d_f32_nhwc (ops.rs:1356-1436) is acc = fma(x, w, acc) over kh,
    # then kw, then ic, each step rounded once.  The oracle must equal that
    # chain evaluated exactly, and the inputs are chosen so that an ic-first
    # chain or a separately rounded multiply and add give other bits.
    r = np.random.default_rng(2024)
    x = r.uniform(-1, 1, (1, 4, 4, 6)).astype(np.float32)
    w = r.uniform(-1, 1, (3, 3, 6, 3)).astype(np.float32)
    ref = _conv_exact(x, w, 1)
    got = oracle.conv2d_f32_nhwc(x, w, (1, 1), (1, 1))
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(oracle.conv2d_f32_nhwc_st(x, w, (1, 1), (1, 1)), ref)
    # the planted mistakes are visible on these inputs
    assert np.any(_conv_exact(x, w, 1, order="ic_kh_kw") != ref)
    assert np.any(_conv_exact(x, w, 1, fused=False) != ref)


def test_round_f32_helper_against_numpy():
    # the rounding helper itself: equal to numpy's double -> float cast on
    # values exactly representable in double, ties and subnormals included
    vals = [1 + 2.0 ** -24, 1 + 3 * 2.0 ** -24, -(1 + 2.0 ** -24), 2.0 ** -149 * 1.5, 2.0 ** -149 * 2.5,
            3.0 * 2.0 ** -130, 0.1, -123456.789]
    for v in vals:
        assert float(_round_f32(Fraction(v))) == float(np.float32(v)), v
