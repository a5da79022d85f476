"""Graph IR builder, compiler passes and the HIP graph runtime.

``Graph`` is the C-ABI form of ``dragonwing_onnx::Graph`` (ops in order,
named tensors, initializers; ``crates/dragonwing-onnx/src/graph.rs:18-31``)
with the passes ``fold_batchnorm``, ``convert_nchw_to_nhwc``,
``apply_fusion_passes``, ``convert_to_f16`` and the QDQ quantizer.
``HipGraphRuntime`` mirrors ``VulkanGraphRuntime``
(``crates/dragonwing-onnx/src/vulkan_runtime.rs:115-469``).
"""
from __future__ import annotations

import ctypes as C
import json

import numpy as np

from ._lib import RELEASE_GRAPH, RELEASE_RUNTIME, DwOpParams, check, load, native_calls_allowed, track

GRAPH_F32, GRAPH_F16, GRAPH_I8, GRAPH_QU8 = 0, 1, 2, 3
DT = {"f32": 0, "f16": 1, "i8": 2, "u8": 3, "i32": 4}
NP_OF_DT = {0: np.float32, 1: np.uint16, 2: np.int8, 3: np.uint8, 4: np.int32}

OP_KIND = {
    "None": 0, "Conv2d": 1, "Add": 2, "Mul": 3, "Sigmoid": 4, "MaxPool": 5, "Concat": 6, "Split": 7,
    "Resize": 8, "BatchNorm": 9, "Requantize": 10, "AddQuantized": 11, "Quantize": 12, "Dequantize": 13,
    "Conv2dRequantReluI8Nhwc": 14, "QLinearConv": 32, "QuantizeLinear": 33, "DequantizeLinear": 34,
    "QLinearAdd": 35, "QLinearLUT": 36, "Gemm": 15, "GlobalAvgPool": 16, "Softmax": 17, "Clip": 18,
    "Reshape": 19, "YoloDetect": 37, "AvgPool": 20, "Sub": 21, "Div": 22, "Transpose": 23, "Slice": 24,
}
# default OpParams kind per op_type
KIND_OF_TYPE = {"Conv": "Conv2d", "Add": "Add", "Mul": "Mul", "Sigmoid": "Sigmoid", "MaxPool": "MaxPool",
                "Concat": "Concat", "Split": "Split", "Resize": "Resize", "BatchNormalization": "BatchNorm",
                "Relu": "None", "SiLU": "None", "Gemm": "Gemm", "MatMul": "None", "Flatten": "None",
                "GlobalAveragePool": "GlobalAvgPool", "Softmax": "Softmax", "Clip": "Clip",
                "Reshape": "Reshape", "Requantize": "Requantize", "AddQuantized": "AddQuantized",
                "Quantize": "Quantize", "Dequantize": "Dequantize",
                "Conv2dRequantReluI8": "Conv2dRequantReluI8Nhwc", "YoloDetect": "YoloDetect",
                "AveragePool": "AvgPool", "Sub": "Sub", "Div": "Div", "Transpose": "Transpose", "Slice": "Slice"}


def _params(kind: str, **kw) -> DwOpParams:
    p = DwOpParams()
    p.kind = OP_KIND[kind]
    p.group = kw.get("group", 1)
    p.dilations[:] = kw.get("dilations", (1, 1))
    if "kernel_shape" in kw:
        p.kernel_shape[:] = kw["kernel_shape"]
    p.strides[:] = kw.get("strides", (1, 1))
    p.pads[:] = kw.get("pads", (0, 0, 0, 0))
    p.axis = kw.get("axis", 0)
    sizes = kw.get("split_sizes", ())
    p.num_splits = len(sizes)
    for i, s in enumerate(sizes):
        p.split_sizes[i] = s
    p.out_h, p.out_w = kw.get("out_hw", (0, 0))
    p.mode_nearest = 1 if kw.get("mode", "nearest") == "nearest" else 0
    p.scale = kw.get("scale", 0.0)
    p.scale_a_over_out = kw.get("scale_a_over_out", 0.0)
    p.scale_b_over_out = kw.get("scale_b_over_out", 0.0)
    p.has_relu = int(kw.get("has_relu", 0))
    p.epsilon = kw.get("epsilon", 1e-5)
    p.act = kw.get("act", 0)
    p.alpha = kw.get("alpha", 1.0)
    p.beta = kw.get("beta", 1.0)
    p.trans_a = int(kw.get("trans_a", 0))
    p.trans_b = int(kw.get("trans_b", 0))
    p.clip_min = kw.get("clip_min", float("-inf"))
    p.clip_max = kw.get("clip_max", float("inf"))
    p.reg_max = int(kw.get("reg_max", 0))
    ls = list(kw.get("level_strides", ()))
    for i, v in enumerate(ls[:4]):
        p.level_strides[i] = float(v)
    for i, v in enumerate(kw.get("perm", ())):
        p.perm[i] = int(v)
    sl = kw.get("slices", ())  # (axis, start, end, step) per sliced axis, resolved
    p.num_slice_axes = len(sl)
    for i, (ax, st, en, sp) in enumerate(sl):
        p.slice_axes[i], p.slice_starts[i], p.slice_ends[i], p.slice_steps[i] = ax, st, en, sp
    return p


def _cstrs(names):
    arr = (C.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
    return arr


class Graph:
    """A compiled-graph IR owned by libdwhip (one ``dw_graph``)."""

    def __init__(self, dtype: int = GRAPH_F32, _handle=None):
        if _handle is None:
            h = C.c_void_p()
            check(load().dw_graph_create(dtype, C.byref(h)))
            _handle = h.value
        self._h = _handle
        track(self, RELEASE_GRAPH)

    @classmethod
    def from_onnx(cls, data: bytes) -> "Graph":
        """The F32 NCHW graph of a serialized ONNX model (QDQ models carry
        their quantization for quantize_qdq)."""
        buf = C.create_string_buffer(bytes(data), len(data))
        h = C.c_void_p()
        check(load().dw_graph_from_onnx(buf, len(data), C.byref(h)))
        return cls(_handle=h.value)

    @property
    def handle(self):
        return self._h

    def _release(self):
        if self._h:
            load().dw_graph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            if native_calls_allowed():
                self._release()
        except Exception:
            pass

    # --- building ---------------------------------------------------------
    def add_tensor(self, name: str, dims, dtype: str = "f32"):
        d = (C.c_int64 * max(1, len(dims)))(*dims)
        check(load().dw_graph_add_tensor(self._h, name.encode(), d, len(dims), DT[dtype]))
        return name

    def set_initializer(self, name: str, data: np.ndarray):
        a = np.ascontiguousarray(data)
        check(load().dw_graph_set_initializer(self._h, name.encode(), a.ctypes.data, a.nbytes))

    def add_initializer(self, name: str, data: np.ndarray, dtype: str = "f32"):
        self.add_tensor(name, data.shape, dtype)
        self.set_initializer(name, data)
        return name

    def set_quant(self, name: str, scale: float, zero_point: int):
        check(load().dw_graph_set_quant(self._h, name.encode(), float(scale), int(zero_point)))

    def set_channel_scales(self, name: str, scales):
        s = np.ascontiguousarray(scales, np.float32)
        check(load().dw_graph_set_channel_scales(self._h, name.encode(), s.ctypes.data, s.size))

    def add_op(self, name: str, op_type: str, inputs, outputs, kind: str | None = None, **kw):
        p = _params(kind or KIND_OF_TYPE.get(op_type, "None"), **kw)
        check(load().dw_graph_add_op(self._h, name.encode(), op_type.encode(), _cstrs(inputs), len(inputs),
                                     _cstrs(outputs), len(outputs), C.byref(p)))

    def set_io(self, inputs, outputs):
        check(load().dw_graph_set_io(self._h, _cstrs(inputs), len(inputs), _cstrs(outputs), len(outputs)))

    # --- passes -----------------------------------------------------------
    def fold_batchnorm(self):
        check(load().dw_graph_fold_batchnorm(self._h))

    def convert_nchw_to_nhwc(self):
        check(load().dw_graph_convert_nchw_to_nhwc(self._h))

    def apply_fusion_passes(self) -> int:
        n = C.c_int(0)
        check(load().dw_graph_apply_fusion_passes(self._h, C.byref(n)))
        return n.value

    def convert_to_f16(self):
        check(load().dw_graph_convert_to_f16(self._h))

    def set_activation_range(self, name: str, lo: float, hi: float):
        check(load().dw_graph_set_activation_range(self._h, name.encode(), float(lo), float(hi)))

    def quantize_qdq(self, keep_f16_ops=()):
        keep = list(keep_f16_ops)
        check(load().dw_graph_quantize_qdq(self._h, _cstrs(keep), len(keep)))

    # --- introspection ----------------------------------------------------
    def to_dict(self) -> dict:
        return json.loads(load().dw_graph_to_json(self._h).decode())

    def initializer(self, name: str, dtype=None, shape=None) -> np.ndarray:
        ptr = C.c_void_p()
        n = C.c_size_t()
        check(load().dw_graph_get_initializer(self._h, name.encode(), C.byref(ptr), C.byref(n)))
        if not ptr.value:
            raise KeyError(f"{name} has no initializer")
        raw = np.frombuffer((C.c_uint8 * n.value).from_address(ptr.value), np.uint8).copy()
        if dtype is not None:
            raw = raw.view(dtype)
        if shape is not None:
            raw = raw.reshape(shape)
        return raw


RT_EXACT_U8_F16_CONV = 1  # DW_RT_EXACT_U8_F16_CONV
RT_EXACT_F16_DEPTHWISE = 2  # DW_RT_EXACT_F16_DEPTHWISE


class HipGraphRuntime:
    """``VulkanGraphRuntime`` on the HIP backend."""

    def __init__(self, graph: Graph, backend, exact_u8_f16: bool = False, exact_f16_dw: bool = False):
        """exact_u8_f16: the convs that read u8 activations and write f16 (a
        QDQ graph's fp16 tail layers) run in the reference's accumulation
        order, bit-identical to the CPU, instead of on the fp16 matrix cores.
        exact_f16_dw: fp16 depthwise convs in the reference's order instead
        of the packed-f16 band kernel."""
        h = C.c_void_p()
        flags = (RT_EXACT_U8_F16_CONV if exact_u8_f16 else 0) | (RT_EXACT_F16_DEPTHWISE if exact_f16_dw else 0)
        check(load().dw_hip_graph_runtime_create_ex(backend.handle, graph.handle, flags, C.byref(h)))
        self._h = h.value
        self._backend = backend  # keeps the backend alive
        track(self, RELEASE_RUNTIME)

    def _release(self):
        if self._h:
            load().dw_hip_graph_runtime_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            if native_calls_allowed():
                self._release()
        except Exception:
            pass

    def close(self):
        self._release()

    def set_input_f32(self, name: str, data):
        a = np.ascontiguousarray(data, np.float32)
        check(load().dw_hip_graph_set_input_f32(self._h, name.encode(), a.ctypes.data, a.size))

    def set_input_bytes(self, name: str, data):
        a = np.ascontiguousarray(data)
        check(load().dw_hip_graph_set_input_bytes(self._h, name.encode(), a.ctypes.data, a.nbytes))

    def set_input_nchw_f32(self, name: str, data):
        """The input as NCHW f32 (before the layout pass); the GPU transposes
        it, or the stem conv reads it directly."""
        a = np.ascontiguousarray(data, np.float32)
        check(load().dw_hip_graph_set_input_nchw_f32(self._h, name.encode(), a.ctypes.data, a.size))

    def bind_input_nchw_f32(self, name: str, buf):
        """Every run reads the input from the device buffer (NCHW f32)."""
        check(load().dw_hip_graph_bind_input_nchw_f32(self._h, name.encode(), buf.handle))

    def run_unbatched(self):
        """run_unbatched (vulkan_runtime.rs:423-470): launches one by one,
        errors name the failing launch; DW_TRACE=1 prints and syncs each."""
        check(load().dw_hip_graph_run_unbatched(self._h))

    def _io(self, which: int):
        lib = load()
        out = []
        for i in range(lib.dw_hip_graph_num_io(self._h, which)):
            name = lib.dw_hip_graph_io_name(self._h, which, i).decode()
            dims = (C.c_int64 * 4)()
            rank = C.c_int()
            check(lib.dw_hip_graph_tensor_shape(self._h, name.encode(), dims, C.byref(rank)))
            out.append((name, tuple(dims[:rank.value])))
        return out

    def inputs(self):
        """Input tensor names and shapes (vulkan_runtime.rs:213-216)."""
        return self._io(0)

    def outputs(self):
        """Output tensor names and shapes (vulkan_runtime.rs:218-221)."""
        return self._io(1)

    def run(self):
        check(load().dw_hip_graph_run(self._h))

    def tensor_bytes(self, name: str) -> int:
        n = C.c_size_t()
        check(load().dw_hip_graph_tensor_bytes(self._h, name.encode(), C.byref(n)))
        return n.value

    def activation_bytes(self) -> tuple[int, int]:
        """(arena bytes, bytes without reuse): the activation arena, in which
        storage whose lifetimes do not overlap shares bytes, and what the
        same storage takes with no sharing (the reference's SlabStats)."""
        a, u = C.c_size_t(), C.c_size_t()
        check(load().dw_hip_graph_activation_bytes(self._h, C.byref(a), C.byref(u)))
        return a.value, u.value

    def get_output_bytes(self, name: str) -> np.ndarray:
        out = np.empty(self.tensor_bytes(name), np.uint8)
        check(load().dw_hip_graph_get_output_bytes(self._h, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def get_output_f32(self, name: str, count: int) -> np.ndarray:
        out = np.empty(count, np.float32)
        check(load().dw_hip_graph_get_output_f32(self._h, name.encode(), out.ctypes.data, count))
        return out

    def enable_capture(self, on: bool = True):
        check(load().dw_hip_graph_enable_capture(self._h, int(on)))

    def launches(self) -> list[dict]:
        """Per-launch kernel name, fused op names, algorithmic ops and bytes."""
        lib = load()
        out = []
        for i in range(lib.dw_hip_graph_num_launches(self._h)):
            parts = lib.dw_hip_graph_launch_info(self._h, i).decode().split(" ")
            out.append({"kernel": parts[0], "ops": " ".join(parts[1:-2]), "work": float(parts[-2]),
                        "bytes": float(parts[-1])})
        return out

    def run_profiled(self) -> np.ndarray:
        n = load().dw_hip_graph_num_launches(self._h)
        ms = np.zeros(n, np.float32)
        check(load().dw_hip_graph_run_profiled(self._h, ms.ctypes.data))
        return ms

    def time_launches(self, repeat: int = 10) -> np.ndarray:
        """Per-launch milliseconds: each launch enqueued `repeat` times back
        to back between one event pair (dw_hip_graph_time_launches); the
        kernel's duration plus the gap between consecutive dispatches."""
        n = load().dw_hip_graph_num_launches(self._h)
        ms = np.zeros(n, np.float32)
        check(load().dw_hip_graph_time_launches(self._h, repeat, ms.ctypes.data))
        return ms


def time_launches_rotated(runtimes, repeat: int = 8) -> np.ndarray:
    """Per-launch milliseconds with the repeats of each launch cycling
    through ``runtimes`` (HipGraphRuntime objects of one graph on one
    backend): dw_hip_graph_time_launches_rotated."""
    lib = load()
    n = lib.dw_hip_graph_num_launches(runtimes[0]._h)
    handles = (C.c_void_p * len(runtimes))(*[rt._h for rt in runtimes])
    ms = np.zeros(n, np.float32)
    check(lib.dw_hip_graph_time_launches_rotated(handles, len(runtimes), repeat, ms.ctypes.data))
    return ms


def calibrate(backend, graph: Graph, input_name: str, images: np.ndarray):
    """Runs the F32 NHWC graph on the GPU over ``images`` ([k*N, H, W, C] f32)
    and stores per-tensor min/max ranges in ``graph``."""
    imgs = np.ascontiguousarray(images, np.float32)
    per = int(np.prod(imgs.shape[1:]))
    check(load().dw_hip_calibrate(backend.handle, graph.handle, input_name.encode(), imgs.ctypes.data, per,
                                  imgs.shape[0]))


def onnx_inspect(data: bytes) -> dict:
    """The parsed model as the loader sees it (nodes, attributes,
    initializers, inputs, outputs, opset)."""
    buf = C.create_string_buffer(bytes(data), len(data))
    need = C.c_size_t()
    check(load().dw_onnx_inspect(buf, len(data), None, 0, C.byref(need)))
    out = C.create_string_buffer(need.value)
    check(load().dw_onnx_inspect(buf, len(data), out, need.value, C.byref(need)))
    return json.loads(out.value.decode())
