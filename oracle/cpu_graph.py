"""CpuGraphRuntime restated over the oracle ops — TEST INFRASTRUCTURE ONLY.

Executes a graph description (the JSON form of the IR: tensors with dims,
dtype and quantization parameters, ops in order) op by op, the way
``CpuGraphRuntime::run`` / ``dispatch_op`` does
(``crates/dragonwing-onnx/src/runtime.rs:874-942``): no fusion, every
intermediate stored in its own dtype, conv bias as a separate pass
(``runtime.rs:1445-1498``), SiLU as Sigmoid then Mul.  The ONNX quantized
ops (QLinearConv, QLinearLUT, QLinearAdd, QuantizeLinear,
DequantizeLinear) and padded MaxPool are the extensions defined in
``oracle/dw_oracle.cpp`` Part B.  Transpose, Slice, Sub, Div, broadcasting
Add / Mul and AveragePool are the numpy restatements of Part D
(``oracle/__init__.py``); LayoutTranspose is the pure byte permutation that
convert_nchw_to_nhwc inserts around a Reshape of a 4-D tensor.

The reference's INT8 form (``QuantizedGraphCompiler``, ``quantize.rs:73-368``,
and fusion pass 3, ``fusion.rs:192-334``) runs with the semantics of the ops
it names, which ``CpuGraphRuntime`` itself refuses (``runtime.rs:934-941``,
``:1497``): an INT8 Conv is ``conv2d_i8_nhwc`` (``ops.rs:3086-3142``) to its
int32 accumulator, Requantize is ``requantize_i32_to_i8`` (``ops.rs:3380-3386``),
Conv2dRequantReluI8 is the three in sequence as
``conv2d_requant_relu_i8_packed`` defines them (``dragonwing-vulkan
ops.rs:2294-2430``), AddQuantized is ``add_i8``, Quantize / Dequantize are
``quantize_f32_to_i8`` / ``dequantize_i8_to_f32``.  The accumulator that
the reference names "<t>_i32" without any op writing it becomes the Conv's
output, and a Concat/Split axis left in NCHW numbering (1) on NHWC tensors
is taken as the channel axis when the shapes are a channel join -- the
same two normalisations the HIP runtime applies.
"""
from __future__ import annotations

import numpy as np

import oracle

F32, F16, I8, U8, I32 = 0, 1, 2, 3, 4
NP = {F32: np.float32, F16: np.uint16, I8: np.int8, U8: np.uint8, I32: np.int32}


class CpuGraph:
    def __init__(self, desc: dict, initializer, threads: int | None = None, int8_threads: int | None = None):
        """desc: Graph.to_dict(); initializer(name, dtype, shape) -> ndarray.
        threads: the _mt ops' thread count; int8_threads: the integer convs'
        (the reference's conv2d_i8_nhwc is single-threaded, ops.rs:3086-3142;
        row-parallel runs give the same integers)."""
        self.d = desc
        self.t = desc["tensors"]
        self.threads = threads or oracle.default_threads()
        self.int8_threads = int8_threads or self.threads
        self.vals: dict[str, np.ndarray] = {}
        for name, ti in self.t.items():
            if ti["init"]:
                self.vals[name] = initializer(name, NP[ti["dtype"]], tuple(ti["dims"]))

    def set_input(self, name: str, arr: np.ndarray):
        ti = self.t[name]
        self.vals[name] = np.ascontiguousarray(arr, NP[ti["dtype"]]).reshape(ti["dims"])

    def run(self, keep: set[str] | None = None):
        for op in self._normalized_ops():
            self._dispatch(op)
        return self.vals

    def _normalized_ops(self):
        ops = [dict(op, inputs=list(op["inputs"]), outputs=list(op["outputs"])) for op in self.d["ops"]]
        for i, rq in enumerate(ops):
            if rq["type"] != "Requantize":
                continue
            src = rq["inputs"][0]
            if any(src in o["outputs"] for o in ops[:i]):
                continue
            for cv in reversed(ops[:i]):
                if cv["type"] == "Conv" and cv["outputs"][0] == rq["outputs"][0]:
                    cv["outputs"][0] = src
                    break
        dims = lambda n: self.t[n]["dims"]
        for op in ops:
            if op["type"] not in ("Concat", "Split") or op["axis"] != 1:
                continue
            parts, whole = (op["inputs"], op["outputs"][0]) if op["type"] == "Concat" else (op["outputs"], op["inputs"][0])
            w = dims(whole)
            if len(w) == 4 and all(len(dims(q)) == 4 and dims(q)[:3] == w[:3] for q in parts) and \
                    sum(dims(q)[3] for q in parts) == w[3]:
                op["axis"] = 3
        return ops

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
                    y = oracle.relu_f32(y) if op.get("has_relu") else y
                else:
                    y = oracle.depthwise_fp16(x, k, s, (p[0], p[1]), self.threads)
                    y = oracle.bias_add_f16(y, b) if b is not None else y
                    y = oracle.relu_fp16(y) if op.get("has_relu") else y
                self.vals[out[0]] = y
                return
            if x.dtype == np.int8:
                if b is not None:
                    raise NotImplementedError("biased INT8 conv")
                self.vals[out[0]] = oracle.conv2d_i8_nhwc(x, w, s, (p[0], p[1]), self.int8_threads)
                return
            if x.dtype == np.float32:
                y = oracle.conv2d_f32_nhwc(x, w, s, (p[0], p[1]), self.threads)
                if b is not None:
                    y = oracle.bias_add_f32(y, b)
                if op.get("has_relu"):  # Conv + Relu from fusion pass 1
                    y = oracle.relu_f32(y)
            else:
                y = oracle.conv2d_fp16_nhwc(x, w, s, (p[0], p[1]), self.threads)
                if b is not None:
                    y = oracle.bias_add_f16(y, b)
                if op.get("has_relu"):
                    y = oracle.relu_fp16(y)
            self.vals[out[0]] = y
        elif ty == "Conv2dRequantReluI8":
            x, w = ins[0], ins[1]
            if len(ins) > 2 and ins[2] is not None:
                raise NotImplementedError("biased INT8 conv")
            s, p = op["strides"], op["pads"]
            y = oracle.requantize_i32_to_i8(oracle.conv2d_i8_nhwc(x, w, s, (p[0], p[1]), self.int8_threads), op["scale"])
            self.vals[out[0]] = oracle.relu_i8(y) if op["has_relu"] else y
        elif ty == "Requantize":
            self.vals[out[0]] = oracle.requantize_i32_to_i8(ins[0], op["scale"])
        elif ty == "AddQuantized":
            self.vals[out[0]] = oracle.add_i8(ins[0], ins[1], op["scale_a_over_out"], op["scale_b_over_out"])
        elif ty == "Quantize":
            self.vals[out[0]] = oracle.quantize_f32_to_i8(ins[0], op["scale"])
        elif ty == "Dequantize":
            self.vals[out[0]] = oracle.dequantize_i8_to_f32(ins[0], op["scale"])
        elif ty == "Clip":
            self.vals[out[0]] = oracle.clip(ins[0], op["clip_min"], op["clip_max"])
        elif ty == "YoloDetect":
            # the exported detect tail (oracle Part C), f16 levels
            if any(x.dtype != np.uint16 for x in ins):
                raise NotImplementedError("YoloDetect on non-f16 inputs")
            nc = ins[0].shape[3] - 4 * op["reg_max"]
            y = oracle.yolo_detect_tail_f16(ins, op["level_strides"][:len(ins)], nc, op["reg_max"])
            self.vals[out[0]] = y.reshape(t[out[0]]["dims"])
        elif ty == "Softmax":
            x = ins[0]
            self.vals[out[0]] = (oracle.softmax_f16 if x.dtype == np.uint16 else oracle.softmax_f32)(x)
        elif ty == "Reshape":
            self.vals[out[0]] = np.ascontiguousarray(ins[0]).reshape(t[out[0]]["dims"])
        elif ty == "QLinearConv":
            x, w = ins[0], ins[1]
            b = ins[2] if len(ins) > 2 else None
            tx, tw, ty_ = t[op["inputs"][0]], t[op["inputs"][1]], t[out[0]]
            s, p = op["strides"], op["pads"]
            self.vals[out[0]] = oracle.qlinearconv_u8s8(
                x, w, b, s, (p[0], p[1]), tx["scale"], tx["zp"], np.array(tw["ch_scales"], np.float32),
                ty_["scale"], ty_["zp"], self.int8_threads)
        elif ty == "QGemm":
            # QLinearConv on a 1x1 kernel over the rows of A; B stored [1][1][k][n]
            a, w = ins[0], ins[1]
            b = ins[2] if len(ins) > 2 else None
            ta, tw, ty_ = t[op["inputs"][0]], t[op["inputs"][1]], t[out[0]]
            k, n = w.shape[2], w.shape[3]
            y = oracle.qgemm_u8s8(a.reshape(-1, k), w.reshape(k, n), b, ta["scale"], ta["zp"],
                                  np.array(tw["ch_scales"], np.float32), ty_["scale"], ty_["zp"])
            self.vals[out[0]] = y.reshape(ty_["dims"])
        elif ty == "QLinearGlobalAveragePool":
            tx, ty_ = t[op["inputs"][0]], t[out[0]]
            y = oracle.qlinear_gap_u8(ins[0], tx["scale"], tx["zp"], ty_["scale"], ty_["zp"])
            self.vals[out[0]] = y.reshape(ty_["dims"])
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
        elif ty in ("Add", "Mul") and ins[0].shape == ins[1].shape:
            fn = {("Add", True): oracle.add_f32, ("Add", False): oracle.add_fp16,
                  ("Mul", True): oracle.mul_f32, ("Mul", False): oracle.mul_fp16}[(ty, ins[0].dtype == np.float32)]
            self.vals[out[0]] = fn(ins[0], ins[1])
        elif ty in ("Add", "Mul", "Sub", "Div"):
            self.vals[out[0]] = oracle.binary(ty, ins[0], ins[1]).reshape(t[out[0]]["dims"])
        elif ty in ("Transpose", "LayoutTranspose"):
            r = ins[0].ndim
            self.vals[out[0]] = oracle.transpose(ins[0], op["perm"][:r], f16_round_trip=ty == "Transpose")
        elif ty == "Slice":
            self.vals[out[0]] = oracle.slice_axes(ins[0], op["slices"])
        elif ty == "AveragePool":
            self.vals[out[0]] = oracle.avgpool2d_nhwc(ins[0], op["kernel_shape"], op["strides"])
        elif ty == "Relu":
            x = ins[0]
            fn = {np.dtype(np.float32): oracle.relu_f32, np.dtype(np.uint16): oracle.relu_fp16,
                  np.dtype(np.int8): oracle.relu_i8}[x.dtype]
            self.vals[out[0]] = fn(x)
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
            if op["axis"] == 3 and ins[0].ndim == 4:
                self.vals[out[0]] = oracle.concat_channels(ins)
            else:  # any other axis of the row-major tensors: the elements in order
                self.vals[out[0]] = np.ascontiguousarray(np.concatenate(ins, axis=op["axis"]))
        elif ty == "Split":
            if op["axis"] == 3 and ins[0].ndim == 4:
                parts = oracle.split_channels(ins[0], op["split_sizes"])
            else:
                cuts = np.cumsum(op["split_sizes"])[:-1]
                parts = [np.ascontiguousarray(v) for v in np.split(ins[0], cuts, axis=op["axis"])]
            for n, v in zip(out, parts):
                self.vals[n] = v
        elif ty == "GlobalAveragePool":
            x = ins[0]
            y = oracle.global_avg_pool_f32(x) if x.dtype == np.float32 else oracle.global_avg_pool_fp16(x)
            self.vals[out[0]] = y.reshape(t[out[0]]["dims"])
        elif ty == "Flatten":
            self.vals[out[0]] = np.ascontiguousarray(ins[0]).reshape(t[out[0]]["dims"])
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


def calibrate(desc: dict, initializer, input_name: str, images: np.ndarray, threads: int | None = None):
    """Calibrator::new / feed / compute_params (crates/dragonwing-onnx/src/
    calibration.rs:90-260) over an F32 NHWC graph: the images run through the
    graph in batches of its N, and after every op each f32 tensor it wrote
    updates that tensor's (min, max) with its finite values only
    (TensorStats::update, calibration.rs:56-63; feed, :170-205).  As in feed,
    only op outputs are recorded, not the graph input.  Returns
    {name: (min, max)}; QuantScale::from_range turns a range into absmax/127.

    Where this departs from calibration.rs:632-830: the ops run with
    CpuGraphRuntime's semantics on the NHWC graph (the conv's kh -> kw -> ic
    chain of fused multiply-adds, the bias pass after it, padded MaxPool),
    i.e. the graph the quantized runtime executes; the reference's
    Calibrator instead indexes its convs as NCHW (ic -> kh -> kw, separate
    multiply and add) and ignores MaxPool padding, which the documented
    pipeline's NHWC graph (docs/yolo-vulkan-pipeline.md:228-240) cannot run.
    """
    if desc["dtype"] != F32:
        raise ValueError("calibration requires an F32 graph")
    t = desc["tensors"]
    batch = t[input_name]["dims"][0]
    images = np.ascontiguousarray(images, np.float32)
    if images.shape[0] % batch:
        raise ValueError("image count must be a multiple of the graph batch")
    cg = CpuGraph(desc, initializer, threads)
    stats: dict[str, tuple[float, float]] = {}
    ops = cg._normalized_ops()
    for i0 in range(0, images.shape[0], batch):
        cg.set_input(input_name, images[i0:i0 + batch])
        for op in ops:
            cg._dispatch(op)
            for o in op["outputs"]:
                if t[o]["init"]:
                    continue
                v = cg.vals[o]
                if v.dtype != np.float32:
                    continue
                f = v[np.isfinite(v)]
                if f.size == 0:
                    continue
                lo, hi = float(f.min()), float(f.max())
                if o in stats:
                    lo, hi = min(stats[o][0], lo), max(stats[o][1], hi)
                stats[o] = (lo, hi)
    return stats
