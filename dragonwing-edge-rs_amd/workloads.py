"""The benchmark workloads as graphs for HipGraphRuntime.

* ``conv_f32``    — Conv2d fp32 + bias + ReLU, N=1, 64->64, 56x56, 3x3 s1 p1
* ``qlinearconv`` — QLinearConv u8 x s8 -> u8, N=32, 80x80x128 -> 40x40x256,
                    3x3 s2 p1, x 0.02/128, y 0.05/128, per-channel weights
* ``dwconv``      — depthwise 3x3 fp16 + bias + SiLU, N=32, C=384, 40x40
* ``yolov8n_f16`` — the YOLOv8n-shaped fp16 graph, batch 32, 640x640
* ``yolov8n_int8``— the same graph u8-quantized (QDQ), batch 32, 640x640

Single-op graphs are written directly in their post-conversion NHWC form
(HWIO weights), the form the dragonwing-onnx passes hand to a runtime.
Each builder returns (graph, inputs, outputs, work) where inputs maps the
input name to the bytes to feed and work describes the algorithmic
operations and bytes of one run.
"""
from __future__ import annotations

import numpy as np

from . import synth
from .graph import GRAPH_F16, GRAPH_F32, GRAPH_QU8, Graph


def conv_f32(index: int = 0):
    x, w, b = synth.conv_f32_case(index)
    n, h, wd, ci = x.shape
    co = w.shape[3]
    g = Graph(GRAPH_F32)
    g.add_tensor("x", x.shape)
    g.add_initializer("w", w)
    g.add_initializer("b", b)
    g.add_tensor("y", (n, h, wd, co))
    g.add_tensor("out", (n, h, wd, co))
    g.add_op("conv", "Conv", ["x", "w", "b"], ["y"], kernel_shape=(3, 3), strides=(1, 1), pads=(1, 1, 1, 1))
    g.add_op("relu", "Relu", ["y"], ["out"])
    g.set_io(["x"], ["out"])
    macs = n * h * wd * co * 9 * ci
    work = {"ops": 2.0 * macs, "bytes": x.nbytes + w.nbytes + b.nbytes + n * h * wd * co * 4,
            "images": n, "dtype": "f32"}
    return g, {"x": x}, ["out"], work, (x, w, b)


def qlinearconv(index: int = 1):
    c = synth.qlinearconv_case(index)
    x, w = c["x"], c["w"]
    n, h, wd, ci = x.shape
    co = w.shape[3]
    ho, wo = (h + 2 - 3) // 2 + 1, (wd + 2 - 3) // 2 + 1
    g = Graph(GRAPH_QU8)
    g.add_tensor("x", x.shape, "u8")
    g.set_quant("x", c["x_scale"], c["x_zp"])
    g.add_initializer("w", w, "i8")
    g.set_channel_scales("w", c["w_scales"])
    g.add_initializer("b", c["bias"], "i32")
    g.add_tensor("y", (n, ho, wo, co), "u8")
    g.set_quant("y", c["y_scale"], c["y_zp"])
    g.add_op("qconv", "QLinearConv", ["x", "w", "b"], ["y"], kind="QLinearConv", kernel_shape=(3, 3),
             strides=(2, 2), pads=(1, 1, 1, 1))
    g.set_io(["x"], ["y"])
    macs = n * ho * wo * co * 9 * ci
    work = {"ops": 2.0 * macs, "bytes": x.nbytes + w.nbytes + c["bias"].nbytes + 4 * co + n * ho * wo * co,
            "images": n, "dtype": "int8"}
    return g, {"x": x}, ["y"], work, c


def dwconv(index: int = 2):
    x, w, b = synth.dwconv_case(index)
    n, h, wd, c = x.shape
    g = Graph(GRAPH_F16)
    g.add_tensor("x", x.shape, "f16")
    g.add_initializer("w", w.reshape(3, 3, 1, c), "f16")
    g.add_initializer("b", b, "f16")
    for t in ("y", "s", "out"):
        g.add_tensor(t, x.shape, "f16")
    g.add_op("dw", "Conv", ["x", "w", "b"], ["y"], kernel_shape=(3, 3), strides=(1, 1), pads=(1, 1, 1, 1),
             group=c)
    g.add_op("sig", "Sigmoid", ["y"], ["s"])
    g.add_op("mul", "Mul", ["y", "s"], ["out"])
    g.set_io(["x"], ["out"])
    work = {"ops": 2.0 * n * h * wd * c * 9, "bytes": 2 * x.nbytes + w.nbytes + b.nbytes, "images": n,
            "dtype": "f16"}
    return g, {"x": x}, ["out"], work, (x, w, b)


def _yolo_work(info):
    # 2 * MACs of the 63 convolutions (8.743 GFLOP per 640x640 image)
    return {"images": info["batch"]}


def yolov8n_f16(batch: int = 32, size: int = 640):
    from . import yolo

    g, info = yolo.f16_graph(batch, size)
    x = yolo.input_images(batch, size)
    return g, {info["input"]: synth.f16_bits(x)}, info["outputs"], dict(_yolo_work(info), dtype="f16"), info


def yolov8n_int8(backend, batch: int = 32, size: int = 640):
    from . import yolo

    g, info = yolo.int8_graph(backend, batch, size)
    x = yolo.input_images(batch, size)
    return g, {info["input"]: synth.f16_bits(x)}, info["outputs"], dict(_yolo_work(info), dtype="int8"), info
