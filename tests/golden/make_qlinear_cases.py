"""Writes qlinear_cases.json: hand-derived fixtures for the ONNX quantized
ops (QLinearConv, QuantizeLinear, QLinearAdd), which dragonwing-edge-rs does
not implement.  Every expected value is computed here with exact integer /
dyadic arithmetic chosen so that results land on .5 ties (round half to even
decides) and on the saturation bounds; nothing is taken from the oracle.

Run:  python tests/golden/make_qlinear_cases.py
"""
import json
from fractions import Fraction
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "qlinear_cases.json"


def rne(fr: Fraction) -> int:
    """Round half to even on an exact rational."""
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        return fl + 1
    return fl


def sat(v: int) -> int:
    return max(0, min(255, v))


def qconv_ref(x, w, bias, stride, pad, x_zp, M, y_zp):
    """Direct evaluation of the ONNX definition in exact integers/rationals."""
    n, h, wd, ci = x.shape
    kh, kw, _, co = w.shape
    ho = (h + 2 * pad - kh) // stride + 1
    wo = (wd + 2 * pad - kw) // stride + 1
    y = np.zeros((n, ho, wo, co), np.int64)
    for b in range(n):
        for oh in range(ho):
            for ow in range(wo):
                for oc in range(co):
                    acc = int(bias[oc])
                    for i in range(kh):
                        for j in range(kw):
                            ih, iw = oh * stride + i - pad, ow * stride + j - pad
                            for c in range(ci):
                                xv = int(x[b, ih, iw, c]) if 0 <= ih < h and 0 <= iw < wd else x_zp
                                acc += (xv - x_zp) * int(w[i, j, c, oc])
                    y[b, oh, ow, oc] = sat(rne(acc * M[oc]) + y_zp)
    return y


def case(name, x, w, bias, stride, pad, x_scale, x_zp, w_scales, y_scale, y_zp):
    # The scales are powers of two so M = x_scale * w_scale / y_scale is exact
    # in f32 and in Fraction.
    M = [Fraction(x_scale) * Fraction(ws) / Fraction(y_scale) for ws in w_scales]
    y = qconv_ref(x, w, bias, stride, pad, x_zp, M, y_zp)
    return {"name": name, "x_shape": list(x.shape), "x": x.ravel().tolist(), "w_shape": list(w.shape),
            "w": w.ravel().tolist(), "bias": list(map(int, bias)), "stride": [stride, stride],
            "pad": [pad, pad], "x_scale": x_scale, "x_zp": x_zp, "w_scales": w_scales,
            "y_scale": y_scale, "y_zp": y_zp, "y": y.ravel().tolist()}


def main():
    qc = []
    # 1) ties: w = 0, acc = bias; M = 0.5 -> 2.5, 3.5, -2.5, -1.5
    x = np.full((1, 1, 1, 16), 129, np.uint8)
    w = np.zeros((1, 1, 16, 4), np.int8)
    qc.append(case("ties_half_even", x, w, [5, 7, -5, -3], 1, 0, 0.5, 128, [1.0] * 4, 1.0, 128))
    # 2) saturation at both ends and exactly at the bounds
    qc.append(case("saturation", x, w, [1000, -1000, 254, -256], 1, 0, 0.5, 128, [1.0] * 4, 1.0, 128))
    # 3) padded taps read the zero point (contribute 0)
    x3 = np.full((1, 1, 1, 16), 39, np.uint8)
    w3 = np.ones((3, 3, 16, 4), np.int8)
    qc.append(case("padding_is_zero_point", x3, w3, [0, 1, 2, 3], 1, 1, 1.0, 37, [1.0] * 4, 1.0, 100))
    # 4) stride 2, pad 1, ragged 3x3 image, signed weights, M = 0.25
    x4 = np.full((1, 3, 3, 16), 128, np.uint8)
    for hh in range(3):
        for ww in range(3):
            x4[0, hh, ww, 0] = 128 + hh * 3 + ww + 1
    w4 = np.zeros((3, 3, 16, 4), np.int8)
    w4[:, :, 0, 0] = 1
    w4[:, :, 0, 1] = -1
    qc.append(case("stride2_pad1_ragged", x4, w4, [0, 0, 9, -9], 2, 1, 0.25, 128, [1.0] * 4, 1.0, 10))
    # 5) per-channel weight scales differ
    x5 = np.full((1, 2, 2, 16), 130, np.uint8)  # x - zp = 2
    w5 = np.ones((1, 1, 16, 4), np.int8)  # acc = 32 per channel
    qc.append(case("per_channel_scales", x5, w5, [0, 0, 0, 0], 1, 0, 1.0, 128,
                   [0.0625, 0.125, 0.078125, 0.015625], 1.0, 128))

    # QuantizeLinear from f16 values that are exact multiples of scale/2.
    s = 0.25
    vals = [0.0, 0.125, 0.375, 0.625, -0.125, -0.375, 100.0, -100.0, 31.875, 32.125]
    ql_y = [sat(rne(Fraction(v) / Fraction(s)) + 128) for v in vals]
    ql = [{"name": "quantize_ties_and_saturation",
           "x_f16_bits": np.array(vals, np.float32).astype(np.float16).view(np.uint16).tolist(),
           "scale": s, "zp": 128, "y": ql_y}]

    # QLinearAdd with ra = rb = 0.5.
    a = [129, 131, 129, 255, 0, 133, 128]
    b = [128, 128, 130, 255, 0, 128, 127]
    qa_y = [sat(rne(Fraction(ai - 128, 2) + Fraction(bi - 128, 2)) + 128) for ai, bi in zip(a, b)]
    qa = [{"name": "qadd_ties", "a": a, "b": b, "sa": 0.5, "za": 128, "sb": 0.5, "zb": 128, "sy": 1.0,
           "zy": 128, "y": qa_y}]

    OUT.write_text(json.dumps({"qlinearconv": qc, "quantize_linear": ql, "qlinear_add": qa}, indent=1))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
