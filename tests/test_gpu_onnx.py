"""ONNX-loaded graphs on the GPU: the YOLOv8n-shaped INT8 graph at its
headline workload (batch 32, 640x640), written as a QDQ ONNX model, loaded
back (dw_graph_from_onnx) and quantized with the model's own scales and
integers, runs bit-identical to the graph it came from; the float model
loaded and taken through the fp16 passes matches the directly built fp16
graph bit for bit."""
import numpy as np
import pytest

import onnx_writer as ox
from dragonwing_edge_rs_amd import yolo
from dragonwing_edge_rs_amd.graph import Graph, HipGraphRuntime

pytestmark = pytest.mark.gpu


def run(g, inp, x, backend):
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(inp, x)
    rt.run()
    return [rt.get_output_bytes(o).copy() for o in g.to_dict()["outputs"]]


def test_qdq_onnx_int8_graph_full_workload(backend):
    g, info = yolo.int8_graph(backend, batch=32, size=640)
    model = ox.export_qdq(g)
    print(f"QDQ model: {len(model) / 1e6:.2f} MB", flush=True)
    g2 = Graph.from_onnx(model)
    g2.convert_nchw_to_nhwc()
    g2.quantize_qdq()
    x = yolo.input_images(32, 640)
    want = run(g, info["input"], x, backend)
    got = run(g2, g2.to_dict()["inputs"][0], x, backend)
    assert len(got) == len(want)
    for a, b in zip(got, want):
        assert a.tobytes() == b.tobytes()


def test_float_onnx_to_f16_graph(backend):
    g0, info = yolo.build_yolov8n(batch=4, size=160)
    g = Graph.from_onnx(ox.export_float_nchw(g0))
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    g.convert_to_f16()
    ref, _ = yolo.f16_graph(batch=4, size=160)
    x = yolo.input_images(4, 160)
    for a, b in zip(run(g, info["input"], x, backend), run(ref, info["input"], x, backend)):
        assert a.tobytes() == b.tobytes()
