"""apply_fusion_passes (crates/dragonwing-onnx/src/fusion.rs:42-348) on the
host, no GPU: the reference's own fusion tests (fusion.rs:444-705) restated
on the C IR, plus the two places where this build keeps what the reference
loses (the ReLU of a fused Conv + Relu, and Mul(x, Sigmoid(x)) with x written
by an op)."""
import numpy as np
import pytest

from dragonwing_edge_rs_amd.graph import GRAPH_F32, GRAPH_I8, Graph


def conv_graph(dtype=GRAPH_F32, group=1, bias=False, relu=True, requant=None):
    """Conv -> (Requantize) -> (Relu), tensors declared NHWC."""
    g = Graph(dtype)
    et = "i8" if dtype == GRAPH_I8 else "f32"
    c = 32 if group > 1 else 16
    g.add_tensor("x", (1, 8, 8, c), et)
    wdt = np.int8 if et == "i8" else np.float32
    g.add_initializer("w", np.ones((3, 3, 1 if group > 1 else c, 16 if group == 1 else c), wdt), et)
    ins = ["x", "w"]
    if bias:
        g.add_initializer("b", np.zeros(16 if group == 1 else c, np.float32 if et == "f32" else np.int32),
                          "f32" if et == "f32" else "i32")
        ins.append("b")
    co = 16 if group == 1 else c
    g.add_tensor("conv_out", (1, 8, 8, co), et)
    g.add_op("conv1", "Conv", ins, ["conv_out"], kernel_shape=(3, 3), pads=(1, 1, 1, 1), group=group)
    last = "conv_out"
    if requant is not None:
        g.add_tensor("conv_out_i32", (1, 8, 8, co), "i32")
        g.add_op("conv1_requant", "Requantize", ["conv_out_i32"], ["conv_out"], scale=requant)
    if relu:
        g.add_tensor("relu_out", (1, 8, 8, co), et)
        g.add_op("relu1", "Relu", ["conv_out"], ["relu_out"])
        last = "relu_out"
    g.set_io(["x"], [last])
    return g


def test_conv_relu_fusion_removes_relu_and_keeps_it_as_a_flag():
    # test_fusion_removes_ops (fusion.rs:664-704): one op left, writing relu_out
    g = conv_graph()
    assert g.apply_fusion_passes() == 1
    ops = g.to_dict()["ops"]
    assert len(ops) == 1
    assert ops[0]["type"] == "Conv" and ops[0]["name"] == "conv1_fused_relu"
    assert ops[0]["outputs"] == ["relu_out"]
    assert ops[0]["has_relu"] == 1  # the reference drops the ReLU here
    assert "conv_out" not in g.to_dict()["tensors"]


def test_conv_requant_relu_i8_fusion():
    # test_conv_requant_relu_i8_fusion (fusion.rs:527-578)
    g = conv_graph(GRAPH_I8, requant=0.0125)
    g.apply_fusion_passes()
    ops = g.to_dict()["ops"]
    assert len(ops) == 1, "should collapse 3 ops to 1"
    f = ops[0]
    assert f["type"] == "Conv2dRequantReluI8" and f["name"] == "conv1_fused_qrelu"
    assert f["outputs"] == ["relu_out"]
    assert f["kernel_shape"] == [3, 3] and f["strides"] == [1, 1] and f["pads"] == [1, 1, 1, 1]
    assert f["dilations"] == [1, 1] and f["group"] == 1
    assert abs(f["scale"] - 0.0125) < 1e-7 and f["has_relu"] == 1


def test_conv_requant_only_fusion():
    # test_conv_requant_only_fusion (fusion.rs:580-622)
    g = conv_graph(GRAPH_I8, relu=False, requant=0.02)
    g.apply_fusion_passes()
    ops = g.to_dict()["ops"]
    assert len(ops) == 1
    assert ops[0]["type"] == "Conv2dRequantReluI8" and ops[0]["outputs"] == ["conv_out"]
    assert ops[0]["has_relu"] == 0


def test_conv_requant_skipped_when_group_ne_1():
    # test_conv_requant_skipped_when_group_ne_1 (fusion.rs:624-662)
    g = conv_graph(GRAPH_I8, group=32, relu=False, requant=0.01)
    before = len(g.to_dict()["ops"])
    g.apply_fusion_passes()
    assert len(g.to_dict()["ops"]) == before


def test_conv_requant_skipped_with_bias():
    # fusion.rs:303-309: a biased INT8 conv is left alone
    g = conv_graph(GRAPH_I8, bias=True, relu=False, requant=0.01)
    g.apply_fusion_passes()
    assert [op["type"] for op in g.to_dict()["ops"]] == ["Conv", "Requantize"]


@pytest.mark.parametrize("order", ["x_first", "s_first"])
@pytest.mark.parametrize("x_written", [False, True])
def test_silu_fusion_either_operand_order(order, x_written):
    # test_silu_detection (fusion.rs:497-525) is Mul(x, sig_out) with x a graph
    # input; here also x written by an op and the swapped operand order.
    g = Graph(GRAPH_F32)
    g.add_tensor("in", (1, 4, 4, 8))
    src = "in"
    if x_written:
        g.add_tensor("x", (1, 4, 4, 8))
        g.add_op("relu0", "Relu", ["in"], ["x"])
        src = "x"
    g.add_tensor("sig_out", (1, 4, 4, 8))
    g.add_tensor("silu_out", (1, 4, 4, 8))
    g.add_op("sigmoid1", "Sigmoid", [src], ["sig_out"])
    ins = [src, "sig_out"] if order == "x_first" else ["sig_out", src]
    g.add_op("mul1", "Mul", ins, ["silu_out"])
    g.set_io(["in"], ["silu_out"])
    assert g.apply_fusion_passes() == 1
    ops = g.to_dict()["ops"]
    assert [op["type"] for op in ops][-1] == "SiLU"
    silu = ops[-1]
    assert silu["name"] == "mul1_silu" and silu["inputs"] == [src] and silu["outputs"] == ["silu_out"]
    assert "Sigmoid" not in [op["type"] for op in ops]


def test_silu_not_fused_when_sigmoid_has_other_readers():
    g = Graph(GRAPH_F32)
    for n in ("x", "s", "y", "z"):
        g.add_tensor(n, (1, 2, 2, 4))
    g.add_op("sig", "Sigmoid", ["x"], ["s"])
    g.add_op("mul", "Mul", ["x", "s"], ["y"])
    g.add_op("relu", "Relu", ["s"], ["z"])
    g.set_io(["x"], ["y", "z"])
    assert g.apply_fusion_passes() == 0
    assert len(g.to_dict()["ops"]) == 3
