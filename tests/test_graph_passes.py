"""Host-side graph compiler (no GPU): the YOLOv8n-shaped builder, BN folding,
NCHW->NHWC, SiLU fusion, f16 conversion and the QDQ quantizer, checked
against the oracle's restatements and closed forms."""
import numpy as np
import pytest

import oracle
from dragonwing_edge_rs_amd import yolo
from dragonwing_edge_rs_amd.graph import GRAPH_F16, GRAPH_QU8, Graph


@pytest.fixture(scope="module")
def small():
    return yolo.build_yolov8n(batch=1, size=64)


def op_types(d):
    out = {}
    for op in d["ops"]:
        out[op["type"]] = out.get(op["type"], 0) + 1
    return out


def test_yolov8n_structure(small):
    g, info = small
    d = g.to_dict()
    assert info["convs"] == 63
    counts = op_types(d)
    assert counts["Conv"] == 63 and counts["BatchNormalization"] == 57
    assert counts["Split"] == 8 and counts["Concat"] == 16 and counts["Add"] == 6
    assert counts["MaxPool"] == 3 and counts["Resize"] == 2
    # weights + biases of the published n-scale model (BN params excluded): 3,151,904 minus
    # BN gamma/beta; the count of conv weights and the 6 head biases:
    nconv = sum(int(np.prod(t["dims"])) for n, t in d["tensors"].items() if n.endswith(".weight") and ".bn." not in n)
    assert 3_000_000 < nconv < 3_200_000
    assert info["out_shapes"] == [(1, 8, 8, 144), (1, 4, 4, 144), (1, 2, 2, 144)]


def test_fold_batchnorm_matches_oracle():
    g, info = yolo.build_yolov8n(batch=1, size=64)
    raw = g.to_dict()
    w = g.initializer("b3.weight", np.float32, tuple(raw["tensors"]["b3.weight"]["dims"]))
    bn = {k: g.initializer(f"b3.bn.{k}", np.float32) for k in ("weight", "bias", "running_mean", "running_var")}
    g.fold_batchnorm()
    d = g.to_dict()
    assert "BatchNormalization" not in op_types(d)
    conv = next(op for op in d["ops"] if op["name"] == "b3")
    assert conv["outputs"] == ["b3.bn_out"] and conv["inputs"][2] == "b3.weight_bias_folded"
    w2 = g.initializer("b3.weight", np.float32, w.shape)
    b2 = g.initializer("b3.weight_bias_folded", np.float32)
    ew, eb = oracle.fold_batchnorm(w, None, bn["weight"], bn["bias"], bn["running_mean"], bn["running_var"], 1e-3)
    np.testing.assert_array_equal(w2, ew)
    np.testing.assert_array_equal(b2, eb)


def test_nhwc_conversion_and_axes():
    g, _ = yolo.build_yolov8n(batch=1, size=64)
    g.fold_batchnorm()
    w = g.initializer("b1.weight", np.float32, (32, 16, 3, 3))
    g.convert_nchw_to_nhwc()
    d = g.to_dict()
    assert d["tensors"]["b1.weight"]["dims"] == [3, 3, 16, 32]
    np.testing.assert_array_equal(g.initializer("b1.weight", np.float32, (3, 3, 16, 32)), w.transpose(2, 3, 1, 0))
    assert d["tensors"]["images"]["dims"] == [1, 64, 64, 3]
    assert all(op["axis"] == 3 for op in d["ops"] if op["type"] in ("Concat", "Split"))


def test_silu_fusion_and_f16():
    g, _ = yolo.build_yolov8n(batch=1, size=64)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    assert g.apply_fusion_passes() == 57
    d = g.to_dict()
    c = op_types(d)
    assert c["SiLU"] == 57 and "Sigmoid" not in c and "Mul" not in c
    w32 = g.initializer("b1.weight", np.float32, (3, 3, 16, 32))
    g.convert_to_f16()
    d = g.to_dict()
    assert d["dtype"] == GRAPH_F16
    np.testing.assert_array_equal(g.initializer("b1.weight", np.uint16, (3, 3, 16, 32)), oracle.f16_from_f32(w32))
    assert all(t["dtype"] == 1 for t in d["tensors"].values() if not t["init"])


def synthetic_ranges(g):
    # Deterministic stand-in for calibration: every activation in [-3, 4].
    for n, t in g.to_dict()["tensors"].items():
        if not t["init"]:
            g.set_activation_range(n, -3.0, 4.0 + 0.001 * (hash(n) % 7))


def test_quantize_qdq_structure():
    g, info = yolo.build_yolov8n(batch=1, size=64)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    w = g.initializer("b3.weight", np.float32, (3, 3, 32, 64))
    b = g.initializer("b3.weight_bias_folded", np.float32)
    synthetic_ranges(g)
    g.quantize_qdq(info["keep_f16"])
    d = g.to_dict()
    assert d["dtype"] == GRAPH_QU8
    c = op_types(d)
    assert c["QLinearConv"] == 56 and c["Conv"] == 7
    assert c["QLinearLUT"] == 57 and c["QLinearAdd"] == 6
    assert c["QuantizeLinear"] == 1 and c["DequantizeLinear"] == 6
    t = d["tensors"]
    # per-channel weights: reference quantizer rounding (quantize.rs:344-368)
    q = g.initializer("b3.weight", np.int8, (3, 3, 32, 64))
    rows = w.reshape(-1, 64).T  # one row per output channel
    eq, es = oracle.quantize_weights_per_channel(rows)
    np.testing.assert_array_equal(q.reshape(-1, 64).T, eq)
    np.testing.assert_array_equal(np.array(t["b3.weight"]["ch_scales"], np.float32), es)
    # int32 bias = rint(b / (x_scale * w_scale))
    xs = t["b1.bn_out"]["scale"] if "b1.bn_out" in t else None
    conv = next(op for op in d["ops"] if op["name"] == "b3")
    xin = t[conv["inputs"][0]]
    bq = g.initializer("b3.weight_bias_folded", np.int32)
    np.testing.assert_array_equal(
        bq, np.rint(b.astype(np.float64) / (np.float32(xin["scale"]) * es).astype(np.float64)).astype(np.int32))
    # concat members share one scale, zero point 128 everywhere
    cat = next(op for op in d["ops"] if op["name"] == "b2.cat")
    scales = {t[i]["scale"] for i in cat["inputs"]} | {t[cat["outputs"][0]]["scale"]}
    assert len(scales) == 1
    assert all(v.get("zp", 128) == 128 for v in t.values() if "scale" in v)
    # kept fp16 convs: the stem and the six head 1x1s
    kept = [op["name"] for op in d["ops"] if op["type"] == "Conv"]
    assert sorted(kept) == sorted(info["keep_f16"])
    assert t["images"]["dtype"] == 1 and all(t[o]["dtype"] == 1 for o in d["outputs"])
    _ = xs


def test_quantize_requires_ranges():
    g, info = yolo.build_yolov8n(batch=1, size=64)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    from dragonwing_edge_rs_amd import HipError
    with pytest.raises(HipError):
        g.quantize_qdq(info["keep_f16"])


def test_graph_builder_errors():
    from dragonwing_edge_rs_amd import HipError
    g = Graph()
    with pytest.raises(HipError):
        g.add_op("x", "Relu", ["missing"], ["also_missing"])
    g.add_tensor("a", (1, 2, 2, 4))
    with pytest.raises(HipError):
        g.set_initializer("a", np.zeros(3, np.float32))
