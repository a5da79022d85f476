"""CpuGraphRuntime restated over the oracle ops — TEST INFRASTRUCTURE ONLY.

Executes a graph description (the JSON form of the IR: tensors with dims,
dtype and quantization parameters, ops in order) op by op, the way
``CpuGraphRuntime::run`` / ``dispatch_op`` does
(``crates/dragonwing-onnx/src/runtime.rs:874-942``): no fusion, every
intermediate stored in its own dtype, conv bias as a separate pass
(``runtime.rs:1445-1498``), SiLU as Sigmoid then Mul.  The ONNX quantized
ops (QLinearConv, QLinearLUT, QLinearAdd, QuantizeLinear,
DequantizeLinear) and padded MaxPool are the extensions defined in
``oracle/dw_oracle.cpp`` Part B.
"""
from __future__ import annotations

import numpy as np

import oracle

F32, F16, I8, U8, I32 = 0, 1, 2, 3, 4
NP = {F32: np.float32, F16: np.uint16, I8: np.int8, U8: np.uint8, I32: np.int32}


class CpuGraph:
    def __init__(self, desc: dict, initializer, threads: int | None = None):
        """desc: Graph.to_dict(); initializer(name, dtype, shape) -> ndarray."""
        self.d = desc
        self.t = desc["tensors"]
        self.threads = threads or oracle.default_threads()
        self.vals: dict[str, np.ndarray] = {}
        for name, ti in self.t.items():
            if ti["init"]:
                self.vals[name] = initializer(name, NP[ti["dtype"]], tuple(ti["dims"]))

    def set_input(self, name: str, arr: np.ndarray):
        ti = self.t[name]
        self.vals[name] = np.ascontiguousarray(arr, NP[ti["dtype"]]).reshape(ti["dims"])

    def run(self, keep: set[str] | None = None):
        for op in self.d["ops"]:
            self._dispatch(op)
        return self.vals

    def _dispatch(self, op):
        ty = op["type"]
        ins = [self.vals[i] if i else None for i in op["inputs"]]
        out = op["outputs"]
        t = self.t
        if ty == "Conv":
            x, w = ins[0], ins[1]
            b = ins[2] if len(ins) > 2 else None
            s, p = op["strides"], op["pads"]
            if op["group"] > 1:
                # dispatch_conv2d depthwise branch (runtime.rs:1412-1421, :1467-1473)
                if op["group"] != x.shape[3]:
                    raise NotImplementedError("grouped conv")
                k = np.ascontiguousarray(w).reshape(w.shape[0], w.shape[1], -1)
                if x.dtype == np.float32:
                    y = oracle.depthwise_f32(x, k, s, (p[0], p[1]), self.threads)
                    y = oracle.bias_add_f32(y, b) if b is not None else y
                else:
                    y = oracle.depthwise_fp16(x, k, s, (p[0], p[1]), self.threads)
                    y = oracle.bias_add_f16(y, b) if b is not None else y
                self.vals[out[0]] = y
                return
            if x.dtype == np.float32:
                y = oracle.conv2d_f32_nhwc(x, w, s, (p[0], p[1]), self.threads)
                if b is not None:
                    y = oracle.bias_add_f32(y, b)
            else:
                y = oracle.conv2d_fp16_nhwc(x, w, s, (p[0], p[1]), self.threads)
                if b is not None:
                    y = oracle.bias_add_f16(y, b)
            self.vals[out[0]] = y
        elif ty == "QLinearConv":
            x, w = ins[0], ins[1]
            b = ins[2] if len(ins) > 2 else None
            tx, tw, ty_ = t[op["inputs"][0]], t[op["inputs"][1]], t[out[0]]
            s, p = op["strides"], op["pads"]
            self.vals[out[0]] = oracle.qlinearconv_u8s8(
                x, w, b, s, (p[0], p[1]), tx["scale"], tx["zp"], np.array(tw["ch_scales"], np.float32),
                ty_["scale"], ty_["zp"], self.threads)
        elif ty == "QLinearLUT":
            tx, ty_ = t[op["inputs"][0]], t[out[0]]
            if op["act"] != 2:
                raise NotImplementedError("only the SiLU table")
            lut = oracle.silu_lut_u8(tx["scale"], tx["zp"], ty_["scale"], ty_["zp"])
            self.vals[out[0]] = oracle.lut_u8(ins[0], lut)
        elif ty == "QLinearAdd":
            ta, tb, ty_ = t[op["inputs"][0]], t[op["inputs"][1]], t[out[0]]
            self.vals[out[0]] = oracle.qlinear_add_u8(ins[0], ins[1], ta["scale"], ta["zp"], tb["scale"],
                                                      tb["zp"], ty_["scale"], ty_["zp"])
        elif ty == "QuantizeLinear":
            ty_ = t[out[0]]
            self.vals[out[0]] = oracle.quantize_linear_f16_u8(ins[0], ty_["scale"], ty_["zp"])
        elif ty == "DequantizeLinear":
            tx = t[op["inputs"][0]]
            self.vals[out[0]] = oracle.dequantize_linear_u8_f16(ins[0], tx["scale"], tx["zp"])
        elif ty == "Sigmoid":
            self.vals[out[0]] = (oracle.sigmoid_f32 if ins[0].dtype == np.float32 else oracle.sigmoid_fp16)(ins[0])
        elif ty == "Mul":
            self.vals[out[0]] = (oracle.mul_f32 if ins[0].dtype == np.float32 else oracle.mul_fp16)(ins[0], ins[1])
        elif ty == "Add":
            self.vals[out[0]] = (oracle.add_f32 if ins[0].dtype == np.float32 else oracle.add_fp16)(ins[0], ins[1])
        elif ty == "Relu":
            self.vals[out[0]] = (oracle.relu_f32 if ins[0].dtype == np.float32 else oracle.relu_fp16)(ins[0])
        elif ty == "SiLU":
            self.vals[out[0]] = (oracle.silu_f32 if ins[0].dtype == np.float32 else oracle.silu_fp16)(ins[0])
        elif ty == "MaxPool":
            k, s, p = op["kernel_shape"], op["strides"], op["pads"]
            self.vals[out[0]] = oracle.maxpool2d_padded(ins[0], k, s, p)
        elif ty == "Resize":
            if not op["mode_nearest"]:
                raise NotImplementedError("linear resize")
            self.vals[out[0]] = oracle.resize_nearest(ins[0], op["out_h"], op["out_w"])
        elif ty == "Concat":
            if op["axis"] != 3:
                raise NotImplementedError("concat axis")
            self.vals[out[0]] = oracle.concat_channels(ins)
        elif ty == "Split":
            if op["axis"] != 3:
                raise NotImplementedError("split axis")
            parts = oracle.split_channels(ins[0], op["split_sizes"])
            for n, v in zip(out, parts):
                self.vals[n] = v
        elif ty == "GlobalAveragePool":
            x = ins[0]
            y = oracle.global_avg_pool_f32(x) if x.dtype == np.float32 else oracle.global_avg_pool_fp16(x)
            self.vals[out[0]] = y.reshape(t[out[0]]["dims"])
        elif ty == "Flatten":
            self.vals[out[0]] = ins[0].reshape(t[out[0]]["dims"])
        elif ty in ("Gemm", "MatMul"):
            # dispatch_gemm (onnx runtime.rs:1178-1275): the fma path without
            # transposes, the unfused one with; then the bias pass
            a, b = ins[0].reshape(-1, ins[0].shape[-1]), ins[1]
            tb = ty == "Gemm" and op.get("trans_b", 0)
            if ty == "Gemm" and op.get("trans_a", 0):
                raise NotImplementedError("Gemm transA")
            f16 = a.dtype == np.uint16
            if tb:
                c = oracle.gemm_tb(a, b)
            else:
                c = oracle.gemm_fp16(a, b) if f16 else oracle.gemm_f32(a, b)
            if len(ins) > 2 and ins[2] is not None:
                bias = np.ascontiguousarray(ins[2]).ravel()
                cols = np.ascontiguousarray(bias[np.arange(c.shape[1]) % bias.size])
                c = oracle.bias_add_f16(c, cols) if f16 else oracle.bias_add_f32(c, cols)
            self.vals[out[0]] = c.reshape(t[out[0]]["dims"])
        else:
            raise NotImplementedError(f"oracle graph: op type {ty}")
