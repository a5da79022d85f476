"""ONNX loading (dw_graph_from_onnx, dw_onnx_inspect) on the CPU.

* the wire format against the reference's own proto tests
  (crates/dragonwing-onnx/src/proto.rs:276-317: varint 150, a field, a
  length-delimited string) and model tests (model.rs:711-745: data types,
  attribute helpers with defaults);
* the encodings a reader must accept: raw_data or typed fields (float_data,
  int64_data, int32_data), packed or unpacked repeated ints, symbolic
  dimensions; malformed input (truncation, unknown wire types) and opsets
  outside 12..20 are refused;
* the YOLOv8n-shaped float graph written as ONNX loads back as the graph it
  came from (ops, parameters, tensors and weights identical), and runs the
  same passes to the same fp16 graph;
* a u8 graph written in QDQ form loads back and, through quantize_qdq with
  the model's own scales and integers, computes the same bytes as the graph
  it came from (checked on the oracle's CpuGraph).
"""
import numpy as np
import pytest

import onnx_writer as ox
import oracle
from dragonwing_edge_rs_amd import HipError, synth, yolo
from dragonwing_edge_rs_amd.graph import Graph, onnx_inspect


def tiny_model(opset=13, producer="dw-tests", ir_version=7, extra_nodes=(), extra_inits=()):
    w = np.arange(2 * 3 * 3 * 3, dtype=np.float32).reshape(2, 3, 3, 3) / 10
    nodes = [ox.node("Conv", ["x", "w"], ["y"], "conv", kernel_shape=[3, 3], pads=[1, 1, 1, 1]),
             ox.node("Relu", ["y"], ["z"], "relu")] + list(extra_nodes)
    return ox.model(nodes, [ox.tensor("w", w)] + list(extra_inits), [ox.value_info("x", [1, 3, 8, 8])],
                    [ox.value_info("z", [1, 2, 8, 8])], opset=opset, producer=producer, ir_version=ir_version)


def test_wire_format_reference_cases():
    # proto.rs:281-317: varint 0x96 0x01 = 150; field 1 (tag 0x08) varint 150;
    # field 2 (tag 0x12) "testing"
    assert ox.varint(150) == bytes([0x96, 0x01]) and ox.f_varint(1, 150) == bytes([0x08, 0x96, 0x01])
    assert ox.f_str(2, "testing") == bytes([0x12, 0x07]) + b"testing"
    m = tiny_model(producer="testing", ir_version=150)
    assert m[:3] == bytes([0x08, 0x96, 0x01]) and m[3:12] == bytes([0x12, 0x07]) + b"testing"
    info = onnx_inspect(m)
    assert info["ir_version"] == 150 and info["producer"] == "testing" and info["opset"] == 13
    assert [n["op"] for n in info["nodes"]] == ["Conv", "Relu"]
    assert info["inputs"] == [{"name": "x", "shape": [1, 3, 8, 8], "dtype": 1}]


def test_attributes_and_names():
    # test_onnx_node_attr_helpers (model.rs:719-745): kernel_shape [3, 3],
    # strides [1, 1], group 1; unnamed nodes are named op_type + first output
    n = ox.node("Conv", ["x", "w"], ["y"], "", kernel_shape=[3, 3], strides=[1, 1], group=1, alpha=0.5,
                mode="nearest", floats=[1.5, -2.0])
    n2 = ox.key(1, 2) + ox.varint(1) + b"x" + ox.key(2, 2) + ox.varint(2) + b"y2" + ox.f_str(4, "Relu") + \
        ox.f_bytes(5, ox.f_str(1, "ints") + ox.f_ints(8, [4, 5, 6], packed=False))
    info = onnx_inspect(ox.model([n, n2], [], [ox.value_info("x", [1, 3, "N", 8])], []))
    a = info["nodes"][0]["attrs"]
    assert a == {"kernel_shape": [3, 3], "strides": [1, 1], "group": 1, "alpha": 0.5, "mode": "nearest",
                 "floats": [1.5, -2.0]}
    assert info["nodes"][0]["name"] == "Conv_y"
    assert info["nodes"][1]["attrs"] == {"ints": [4, 5, 6]} and info["nodes"][1]["name"] == "Relu_y2"
    assert info["inputs"][0]["shape"] == [1, 3, -1, 8]  # a symbolic dimension is dynamic


@pytest.mark.parametrize("raw,packed", [(True, True), (False, True), (False, False)])
def test_tensor_encodings(raw, packed):
    arrs = {"f": np.linspace(-1, 1, 12, dtype=np.float32).reshape(3, 4),
            "i64": np.array([3, -1, 0, 1 << 40], np.int64),
            "u8": np.array([0, 7, 255, 128], np.uint8),
            "i32": np.array([-5, 2 ** 30, 0], np.int32)}
    inits = [ox.tensor(k, v, raw=raw, packed_dims=packed) for k, v in arrs.items()]
    info = onnx_inspect(ox.model([], inits, [], []))
    got = {t["name"]: t for t in info["initializers"]}
    for k, v in arrs.items():
        assert got[k]["dims"] == list(v.shape) and got[k]["bytes"] == v.nbytes, k


def test_malformed_and_unsupported():
    m = tiny_model()
    with pytest.raises(HipError):
        onnx_inspect(m[:len(m) // 2])  # truncated inside a length-delimited field
    with pytest.raises(HipError):
        onnx_inspect(m + bytes([0x0B]))  # field 1, wire type 3 (groups are not ONNX)
    for bad in (11, 21):
        with pytest.raises(HipError):
            onnx_inspect(tiny_model(opset=bad))
    for ok in (12, 20):
        assert onnx_inspect(tiny_model(opset=ok))["opset"] == ok
    with pytest.raises(HipError):  # a dynamic input dimension cannot be planned
        Graph.from_onnx(ox.model([ox.node("Relu", ["x"], ["y"])], [], [ox.value_info("x", [1, 3, "H", 8])],
                                 [ox.value_info("y", [1, 3, 8, 8])]))
    with pytest.raises(HipError):  # an op type this backend does not run
        Graph.from_onnx(ox.model([ox.node("LSTM", ["x"], ["y"])], [], [ox.value_info("x", [1, 3, 8, 8])],
                                 [ox.value_info("y", [1, 3, 8, 8])]))


def test_tiny_model_builds():
    g = Graph.from_onnx(tiny_model())
    d = g.to_dict()
    assert [op["type"] for op in d["ops"]] == ["Conv", "Relu"]
    assert d["tensors"]["y"]["dims"] == [1, 2, 8, 8] and d["ops"][0]["pads"] == [1, 1, 1, 1]
    np.testing.assert_array_equal(g.initializer("w", np.float32, (2, 3, 3, 3)),
                                  np.arange(54, dtype=np.float32).reshape(2, 3, 3, 3) / 10)


def graph_equal(a: Graph, b: Graph, names=True):
    da, db = a.to_dict(), b.to_dict()
    assert da["dtype"] == db["dtype"]
    assert len(da["ops"]) == len(db["ops"])
    for oa, ob in zip(da["ops"], db["ops"]):
        for k in oa:
            if k in ("name",) and not names:
                continue
            assert oa[k] == ob[k], (oa["name"], k, oa[k], ob[k])
    ta, tb = da["tensors"], db["tensors"]
    assert set(ta) == set(tb)
    for n in ta:
        assert ta[n] == tb[n], n
        if ta[n]["init"]:
            es = {0: 4, 1: 2, 2: 1, 3: 1, 4: 4}[ta[n]["dtype"]]
            ba = a.initializer(n, np.uint8, (int(np.prod(ta[n]["dims"])) * es,))
            bb = b.initializer(n, np.uint8, (int(np.prod(tb[n]["dims"])) * es,))
            np.testing.assert_array_equal(ba, bb, err_msg=n)
    assert da["inputs"] == db["inputs"] and da["outputs"] == db["outputs"]


def test_yolov8n_float_export_loads_back():
    g, info = yolo.build_yolov8n(batch=2, size=64)
    m = ox.export_float_nchw(g)
    g2 = Graph.from_onnx(m)
    graph_equal(g2, g)
    for gg in (g, g2):
        gg.fold_batchnorm()
        gg.convert_nchw_to_nhwc()
        gg.convert_to_f16()
    graph_equal(g2, g)


def oracle_outputs(g, x_f16):
    from oracle.cpu_graph import CpuGraph
    d = g.to_dict()
    cg = CpuGraph(d, g.initializer)
    cg.set_input(d["inputs"][0], x_f16)
    vals = cg.run()
    return [vals[o] for o in d["outputs"]]


def qdq_round_trip(size, batch):
    """(original u8 graph, the same graph exported as QDQ ONNX and loaded
    back through quantize_qdq), with ranges from the oracle Calibrator."""
    from oracle.cpu_graph import calibrate
    gc, info = yolo.calibration_graph(2, size)
    ranges = calibrate(gc.to_dict(), gc.initializer, info["input"], yolo.calibration_images(2, size))
    g, info = yolo.int8_graph_from_ranges(ranges, batch=batch, size=size)
    g2 = Graph.from_onnx(ox.export_qdq(g))
    g2.convert_nchw_to_nhwc()
    g2.quantize_qdq()
    return g, g2, info


def test_qdq_model_computes_the_same_bytes():
    g, g2, info = qdq_round_trip(64, 1)
    t1 = [op["type"] for op in g.to_dict()["ops"]]
    t2 = [op["type"] for op in g2.to_dict()["ops"]]
    assert sorted(t1) == sorted(t2), (sorted(set(t1) ^ set(t2)))
    x = synth.f16_bits(yolo.input_images(1, 64))
    for a, b in zip(oracle_outputs(g, x), oracle_outputs(g2, x)):
        np.testing.assert_array_equal(a, b)


def bad_tensor(name, dims, dtype, payload: bytes) -> bytes:
    """A TensorProto whose declared dims do not match its raw payload."""
    return ox.f_ints(1, dims) + ox.f_varint(2, dtype) + ox.f_bytes(9, payload) + ox.f_str(8, name)


def clip_model(inits, zp_node=None):
    nodes = [ox.node("Clip", ["x", "lo", "hi"], ["y"], "clip")]
    return ox.model(nodes, inits, [ox.value_info("x", [1, 3, 8, 8])], [ox.value_info("y", [1, 3, 8, 8])])


@pytest.mark.parametrize("case", ["float_dims_too_large", "float_short_payload", "negative_dim",
                                  "overflowing_dims", "int64_shape", "dq_int8_weight", "empty_zero_point"])
def test_constant_payload_must_match_dims(case):
    # Every constant the builder reads is checked against the element count
    # its dims declare before it is read; a mismatch is DW_ERR_INVALID (a
    # malformed model), never a read past the payload.
    hi = ox.tensor("hi", np.array([6.0], np.float32))
    four = np.float32(0.0).tobytes()
    if case in ("float_dims_too_large", "float_short_payload", "negative_dim", "overflowing_dims"):
        dims = {"float_dims_too_large": [1 << 26], "float_short_payload": [2], "negative_dim": [-1],
                "overflowing_dims": [1 << 31, 1 << 31, 1 << 31]}[case]
        m = clip_model([bad_tensor("lo", dims, ox.FLOAT, four), hi])
    elif case == "int64_shape":
        nodes = [ox.node("Reshape", ["x", "shape"], ["y"], "r")]
        m = ox.model(nodes, [bad_tensor("shape", [1 << 20], 7, np.int64(2).tobytes() * 2)],
                     [ox.value_info("x", [1, 3, 8, 8])], [ox.value_info("y", [1, 192])])
    elif case == "dq_int8_weight":
        nodes = [ox.node("DequantizeLinear", ["wq", "ws"], ["w"], "dq"),
                 ox.node("Conv", ["x", "w"], ["y"], "conv", kernel_shape=[3, 3], pads=[1, 1, 1, 1])]
        m = ox.model(nodes, [bad_tensor("wq", [2, 3, 3, 3], 3, bytes(10)),
                             ox.tensor("ws", np.array([0.1], np.float32))],
                     [ox.value_info("x", [1, 3, 8, 8])], [ox.value_info("y", [1, 2, 8, 8])])
    else:  # a scalar u8 zero point with no bytes
        nodes = [ox.node("QuantizeLinear", ["x", "s", "zp"], ["xq"], "q"),
                 ox.node("DequantizeLinear", ["xq", "s", "zp"], ["xd"], "dq"),
                 ox.node("Relu", ["xd"], ["y"], "relu")]
        m = ox.model(nodes, [ox.tensor("s", np.array(0.1, np.float32)), bad_tensor("zp", [], 2, b"")],
                     [ox.value_info("x", [1, 3, 8, 8])], [ox.value_info("y", [1, 3, 8, 8])])
    with pytest.raises(HipError) as e:
        Graph.from_onnx(m)
    assert e.value.code == -4, (case, e.value.code, str(e.value))  # DW_ERR_INVALID


def tail_run_on_oracle(size=64, shape_ops=False):
    """The YOLOv8n-shaped float model with the exported detect tail, loaded
    (dw_graph_from_onnx), through fold_batchnorm and convert_nchw_to_nhwc,
    run on the oracle's CpuGraph: (graph, output0 [1, 84, A], the three
    head tensors in NCHW)."""
    from oracle.cpu_graph import CpuGraph
    g0, info = yolo.build_yolov8n(batch=1, size=size)
    g = Graph.from_onnx(ox.export_float_nchw_with_tail(g0, shape_ops=shape_ops, keep_heads=True))
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    d = g.to_dict()
    cg = CpuGraph(d, g.initializer)
    cg.set_input(d["inputs"][0], yolo.input_images(1, size))
    vals = cg.run()
    heads = [np.ascontiguousarray(vals[h].transpose(0, 3, 1, 2)) for h in d["outputs"][1:]]
    return g, vals["output0"], heads


def test_exported_tail_loads_and_computes_the_onnx_meaning():
    # the exported tail (Reshape, Concat, Split, Transpose, Softmax, Conv,
    # Slice, Sub, Add, Div, Mul, Sigmoid, Concat) after convert_nchw_to_nhwc
    # computes what the NCHW ONNX graph means: the f64 statement of the same
    # graph on the same head outputs
    g, out, heads = tail_run_on_oracle()
    ref = ox.tail_reference_nchw(heads)
    assert out.shape == ref.shape == (1, 84, 8 * 8 + 4 * 4 + 2 * 2)
    box, cls = np.abs(out[:, :4] - ref[:, :4]), np.abs(out[:, 4:] - ref[:, 4:])
    assert box.max() <= 1e-5 * np.abs(ref[:, :4]).max() and cls.max() <= 1e-6, (box.max(), cls.max())
    types = [op["type"] for op in g.to_dict()["ops"]]
    for ty in ("Transpose", "Slice", "Sub", "Div", "LayoutTranspose"):
        assert ty in types, ty
    # the layout transposes sit where a Reshape reads an NHWC tensor
    assert types.count("LayoutTranspose") == 4  # three heads and the DFL's 4-D reshape


def test_exported_tail_shape_ops_fold_to_constants():
    # Shape -> Gather -> Unsqueeze -> Concat chains for the Reshape shapes
    # (unsimplified exports) fold into constants: the same ops, same result
    g1, out1, _ = tail_run_on_oracle(shape_ops=False)
    g2, out2, _ = tail_run_on_oracle(shape_ops=True)
    t1 = [op["type"] for op in g1.to_dict()["ops"]]
    t2 = [op["type"] for op in g2.to_dict()["ops"]]
    assert t1 == t2 and "Shape" not in t2 and "Gather" not in t2
    np.testing.assert_array_equal(out1, out2)


def test_pad_folds_into_conv_and_avgpool_loads():
    w = np.arange(2 * 3 * 3 * 3, dtype=np.float32).reshape(2, 3, 3, 3) / 10
    nodes = [ox.node("Pad", ["x", "pads"], ["xp"], "pad"),
             ox.node("Conv", ["xp", "w"], ["y"], "conv", kernel_shape=[3, 3]),
             ox.node("AveragePool", ["y"], ["z"], "pool", kernel_shape=[2, 2], strides=[2, 2])]
    m = ox.model(nodes, [ox.tensor("w", w), ox.tensor("pads", np.array([0, 0, 1, 2, 0, 0, 1, 0], np.int64))],
                 [ox.value_info("x", [1, 3, 8, 8])], [ox.value_info("z", [1, 2, 4, 4])], opset=17)
    d = Graph.from_onnx(m).to_dict()
    assert [op["type"] for op in d["ops"]] == ["Conv", "AveragePool"]
    assert d["ops"][0]["pads"] == [1, 2, 1, 0] and d["tensors"]["y"]["dims"] == [1, 2, 8, 9 - 1]
    bad = ox.model([ox.node("Pad", ["x", "pads"], ["xp"], "pad"), ox.node("Relu", ["xp"], ["y"], "relu")],
                   [ox.tensor("pads", np.array([0, 0, 1, 1, 0, 0, 1, 1], np.int64))],
                   [ox.value_info("x", [1, 3, 8, 8])], [ox.value_info("y", [1, 3, 10, 10])], opset=17)
    with pytest.raises(HipError):  # a Pad that no Conv reads
        Graph.from_onnx(bad)


def test_exported_tail_int8_graph_on_oracle():
    # quantize_qdq of the exported model: the INT8 body as before, the tail
    # after the fp16 head convs stays f16 (with the DFL conv kept fp16), and
    # the u8 graph's output is the f16 statement of the same tail
    from oracle.cpu_graph import CpuGraph, calibrate
    g0, info = yolo.build_yolov8n(batch=1, size=64)
    model = ox.export_float_nchw_with_tail(g0, keep_heads=True)
    gc = Graph.from_onnx(model)
    gc.fold_batchnorm()
    gc.convert_nchw_to_nhwc()
    dc = gc.to_dict()
    ranges = calibrate(dc, gc.initializer, dc["inputs"][0], yolo.calibration_images(2, 64))
    gq = Graph.from_onnx(model)
    gq.fold_batchnorm()
    gq.convert_nchw_to_nhwc()
    for n, (lo, hi) in ranges.items():
        gq.set_activation_range(n, lo, hi)
    gq.quantize_qdq(list(info["keep_f16"]) + ["tail.dfl.conv"])
    d = gq.to_dict()
    t = d["tensors"]
    assert t["output0"]["dtype"] == 1 and t["tail.dfl.p"]["dtype"] == 1
    assert sum(op["type"] == "QLinearConv" for op in d["ops"]) == 56
    cg = CpuGraph(d, gq.initializer)
    cg.set_input(d["inputs"][0], synth.f16_bits(yolo.input_images(1, 64)))
    vals = cg.run()
    out = oracle.f16_to_f32(vals["output0"])
    heads = [vals[h] for h in d["outputs"][1:]]
    fused = oracle.yolo_detect_tail_f16(heads, (8, 16, 32))
    box = np.max(np.abs(out[:, :4] - fused[:, :4])) / np.max(np.abs(fused[:, :4]))
    assert box <= 1e-2 and np.max(np.abs(out[:, 4:] - fused[:, 4:])) <= 1e-2
