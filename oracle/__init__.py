"""dragonwing-cpu oracle — TEST INFRASTRUCTURE ONLY.

numpy-level access to ``oracle/dw_oracle.cpp``, the CPU restatement of the
dragonwing-edge-rs hot-path algorithms (``crates/dragonwing-cpu/src/ops.rs``,
``crates/dragonwing-core/src/dtype.rs``, ``crates/dragonwing-onnx/src/runtime.rs``)
plus the ONNX quantized extensions the reference lacks.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may use
this package, and only as the checker or the timed CPU baseline — never as
part of the product path.

Parity status of each function is recorded in the test that pins it
(``tests/test_oracle_*.py``).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBPATH = HERE / "build" / "libdworacle.so"

_lib = None


def build() -> Path:
    """Compiles the oracle with its Makefile (g++ -O3, no contraction)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBPATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIBPATH.exists():
            build()
        _lib = C.CDLL(str(LIBPATH))
        _declare(_lib)
    return _lib


_P = C.c_void_p
_Z = C.c_size_t
_F = C.c_float
_I = C.c_int


def _declare(L: C.CDLL) -> None:
    sig = {
        "dwo_f16_from_f32": (C.c_uint16, [_F]),
        "dwo_f16_to_f32": (_F, [C.c_uint16]),
        "dwo_f32_to_f16_array": (None, [_P, _P, _Z]),
        "dwo_f16_to_f32_array": (None, [_P, _P, _Z]),
        "dwo_num_cpus": (_I, []),
        "dwo_conv2d_f32_nhwc": (None, [_P, _P, _P] + [_Z] * 11),
        "dwo_conv2d_f32_nhwc_mt": (None, [_P, _P, _P] + [_Z] * 11 + [_I]),
        "dwo_conv2d_fp16_nhwc_mt": (None, [_P, _P, _P] + [_Z] * 11 + [_I]),
        "dwo_depthwise_conv2d_f32_nhwc_mt": (None, [_P, _P, _P] + [_Z] * 11 + [_I]),
        "dwo_depthwise_conv2d_fp16_nhwc_mt": (None, [_P, _P, _P] + [_Z] * 11 + [_I]),
        "dwo_conv2d_i8_nhwc": (None, [_P, _P, _P] + [_Z] * 11),
        "dwo_conv2d_i8_nhwc_rowpar": (None, [_P, _P, _P] + [_Z] * 11 + [_I]),
        "dwo_bias_add_f32_nhwc": (None, [_P, _P, _Z, _Z]),
        "dwo_bias_add_f16_nhwc": (None, [_P, _P, _Z, _Z]),
        "dwo_relu_f32": (None, [_P, _P, _Z]),
        "dwo_relu_fp16": (None, [_P, _P, _Z]),
        "dwo_add_f32": (None, [_P, _P, _P, _Z]),
        "dwo_add_fp16": (None, [_P, _P, _P, _Z]),
        "dwo_mul_f32": (None, [_P, _P, _P, _Z]),
        "dwo_mul_fp16": (None, [_P, _P, _P, _Z]),
        "dwo_sigmoid_f32": (None, [_P, _P, _Z]),
        "dwo_sigmoid_fp16": (None, [_P, _P, _Z]),
        "dwo_requantize_i32_to_i8": (None, [_P, _P, _Z, _F]),
        "dwo_quantize_f32_to_i8": (None, [_P, _P, _Z, _F]),
        "dwo_dequantize_i8_to_f32": (None, [_P, _P, _Z, _F]),
        "dwo_add_i8": (None, [_P, _P, _P, _Z, _F, _F]),
        "dwo_relu_i8": (None, [_P, _P, _Z]),
        "dwo_scale_from_range": (_F, [_F, _F]),
        "dwo_quantize_weights_per_channel": (None, [_P, _P, _P, _Z, _Z]),
        "dwo_maxpool2d_f32_nhwc": (None, [_P, _P] + [_Z] * 8),
        "dwo_resize_nearest_nhwc": (None, [_P, _P] + [_Z] * 7),
        "dwo_concat_channels": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_split_channels": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_fold_batchnorm": (None, [_P, _P, _P, _P, _P, _P, _P, _F, _Z, _Z]),
        "dwo_qlinearconv_u8s8": (None, [_P, _P, _P, _P] + [_Z] * 11 + [_F, _I, _P, _F, _I, _I]),
        "dwo_quantize_linear_f16_u8": (None, [_P, _P, _Z, _F, _I]),
        "dwo_dequantize_linear_u8_f16": (None, [_P, _P, _Z, _F, _I]),
        "dwo_qlinear_add_u8": (None, [_P, _P, _P, _Z, _F, _I, _F, _I, _F, _I]),
        "dwo_silu_lut_u8": (None, [_P, _F, _I, _F, _I]),
        "dwo_lut_u8": (None, [_P, _P, _Z, _P]),
        "dwo_maxpool2d_padded_nhwc": (None, [_P, _P] + [_Z] * 13),
        "dwo_gemm_f32": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_gemm_fp16": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_gemm_i8": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_gemm_f32_tb": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_gemm_fp16_tb": (None, [_P, _P, _P, _Z, _Z, _Z]),
        "dwo_global_avg_pool_f32": (None, [_P, _P, _Z, _Z, _Z, _Z]),
        "dwo_global_avg_pool_fp16": (None, [_P, _P, _Z, _Z, _Z, _Z]),
        "dwo_softmax_f32": (None, [_P, _P, _Z, _Z]),
        "dwo_yolo_detect_tail_f16": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
        "dwo_iou": (_F, [_P, _P]),
        "dwo_qlinear_gap_u8": (None, [_P, _P, _Z, _Z, _Z, _Z, _F, _I, _F, _I]),
        "dwo_yolo_postprocess": (None, [_P, _P, _P, _Z, _Z, _Z, C.c_uint32, C.c_uint32, _F, _F, _I, _Z]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def num_cpus() -> int:
    return lib().dwo_num_cpus()


def default_threads() -> int:
    """Threads for the oracle's row-parallel loops: the online CPUs, at most
    OMP_NUM_THREADS (default 16), the CPU share a one-GPU host gives a job."""
    cap = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(num_cpus(), cap))


# --- F16 -------------------------------------------------------------------
def f16_from_f32(x) -> np.ndarray:
    """F16::from_f32_soft bits (dtype.rs:164-222) of every element."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().dwo_f32_to_f16_array(_p(x), _p(y), x.size)
    return y


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().dwo_f16_to_f32_array(_p(h), _p(y), h.size)
    return y


def out_hw(h, w, kh, kw, sh, sw, ph, pw):
    return (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1


# --- convolutions (NHWC input, HWIO kernel) --------------------------------
def conv2d_f32_nhwc(x, k, stride=(1, 1), pad=(0, 0), threads=None):
    """conv2d_f32_nhwc_mt (ops.rs:1756-1837)."""
    x = np.ascontiguousarray(x, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    n, h, w, ci = x.shape
    kh, kw, ci2, co = k.shape
    assert ci == ci2
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, co), np.float32)
    lib().dwo_conv2d_f32_nhwc_mt(_p(y), _p(x), _p(k), n, h, w, ci, co, kh, kw, stride[0], stride[1],
                                 pad[0], pad[1], threads or default_threads())
    return y


def conv2d_f32_nhwc_st(x, k, stride=(1, 1), pad=(0, 0)):
    """conv2d_f32_nhwc (ops.rs:1356-1436), single thread."""
    x = np.ascontiguousarray(x, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    n, h, w, ci = x.shape
    kh, kw, _, co = k.shape
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, co), np.float32)
    lib().dwo_conv2d_f32_nhwc(_p(y), _p(x), _p(k), n, h, w, ci, co, kh, kw, stride[0], stride[1],
                              pad[0], pad[1])
    return y


def conv2d_fp16_nhwc(xh, kh_, stride=(1, 1), pad=(0, 0), threads=None):
    """conv2d_fp16_nhwc_mt (ops.rs:2572-2651) on f16 bit arrays."""
    xh = np.ascontiguousarray(xh, np.uint16)
    kh_ = np.ascontiguousarray(kh_, np.uint16)
    n, h, w, ci = xh.shape
    kh, kw, _, co = kh_.shape
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, co), np.uint16)
    lib().dwo_conv2d_fp16_nhwc_mt(_p(y), _p(xh), _p(kh_), n, h, w, ci, co, kh, kw, stride[0], stride[1],
                                  pad[0], pad[1], threads or default_threads())
    return y


def depthwise_f32(x, k, stride=(1, 1), pad=(0, 0), threads=None):
    """depthwise_conv2d_f32_nhwc_mt (ops.rs:2734-2815), kernel [kh][kw][c] (multiplier 1)."""
    x = np.ascontiguousarray(x, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    n, h, w, c = x.shape
    kh, kw = k.shape[:2]
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, c), np.float32)
    lib().dwo_depthwise_conv2d_f32_nhwc_mt(_p(y), _p(x), _p(k), n, h, w, c, 1, kh, kw, stride[0],
                                           stride[1], pad[0], pad[1], threads or default_threads())
    return y


def depthwise_fp16(xh, kh_, stride=(1, 1), pad=(0, 0), threads=None):
    """depthwise_conv2d_fp16_nhwc_mt (ops.rs:2819-2933), multiplier 1."""
    xh = np.ascontiguousarray(xh, np.uint16)
    kh_ = np.ascontiguousarray(kh_, np.uint16)
    n, h, w, c = xh.shape
    kh, kw = kh_.shape[:2]
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, c), np.uint16)
    lib().dwo_depthwise_conv2d_fp16_nhwc_mt(_p(y), _p(xh), _p(kh_), n, h, w, c, 1, kh, kw, stride[0],
                                            stride[1], pad[0], pad[1], threads or default_threads())
    return y


def conv2d_i8_nhwc(x, k, stride=(1, 1), pad=(0, 0), threads=1):
    """conv2d_i8_nhwc (ops.rs:3086-3142); threads>1 uses the bit-identical row-parallel variant."""
    x = np.ascontiguousarray(x, np.int8)
    k = np.ascontiguousarray(k, np.int8)
    n, h, w, ci = x.shape
    kh, kw, _, co = k.shape
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, co), np.int32)
    if threads == 1:
        lib().dwo_conv2d_i8_nhwc(_p(y), _p(x), _p(k), n, h, w, ci, co, kh, kw, stride[0], stride[1],
                                 pad[0], pad[1])
    else:
        lib().dwo_conv2d_i8_nhwc_rowpar(_p(y), _p(x), _p(k), n, h, w, ci, co, kh, kw, stride[0],
                                        stride[1], pad[0], pad[1], threads)
    return y


def qlinearconv_u8s8(x, k, bias, stride, pad, x_scale, x_zp, w_scales, y_scale, y_zp, threads=None):
    """ONNX QLinearConv u8 x s8 -> u8 (extension; brute force by definition)."""
    x = np.ascontiguousarray(x, np.uint8)
    k = np.ascontiguousarray(k, np.int8)
    ws = np.ascontiguousarray(w_scales, np.float32)
    n, h, w, ci = x.shape
    kh, kw, _, co = k.shape
    ho, wo = out_hw(h, w, kh, kw, stride[0], stride[1], pad[0], pad[1])
    y = np.empty((n, ho, wo, co), np.uint8)
    bp = 0
    if bias is not None:
        bias = np.ascontiguousarray(bias, np.int32)
        bp = _p(bias)
    lib().dwo_qlinearconv_u8s8(_p(y), _p(x), _p(k), bp, n, h, w, ci, co, kh, kw, stride[0], stride[1],
                               pad[0], pad[1], float(x_scale), int(x_zp), _p(ws), float(y_scale),
                               int(y_zp), threads or default_threads())
    return y


# --- runtime bias passes and elementwise -----------------------------------
def bias_add_f32(y, b):
    y = np.ascontiguousarray(y, np.float32).copy()
    b = np.ascontiguousarray(b, np.float32)
    lib().dwo_bias_add_f32_nhwc(_p(y), _p(b), y.size // b.size, b.size)
    return y


def bias_add_f16(yh, bh):
    yh = np.ascontiguousarray(yh, np.uint16).copy()
    bh = np.ascontiguousarray(bh, np.uint16)
    lib().dwo_bias_add_f16_nhwc(_p(yh), _p(bh), yh.size // bh.size, bh.size)
    return yh


def _unary(fn, x, dt):
    x = np.ascontiguousarray(x, dt)
    y = np.empty_like(x)
    getattr(lib(), fn)(_p(y), _p(x), x.size)
    return y


def _binary(fn, a, b, dt):
    a = np.ascontiguousarray(a, dt)
    b = np.ascontiguousarray(b, dt)
    assert a.shape == b.shape
    y = np.empty_like(a)
    getattr(lib(), fn)(_p(y), _p(a), _p(b), a.size)
    return y


def relu_f32(x): return _unary("dwo_relu_f32", x, np.float32)
def relu_fp16(x): return _unary("dwo_relu_fp16", x, np.uint16)
def sigmoid_f32(x): return _unary("dwo_sigmoid_f32", x, np.float32)
def sigmoid_fp16(x): return _unary("dwo_sigmoid_fp16", x, np.uint16)
def relu_i8(x): return _unary("dwo_relu_i8", x, np.int8)
def add_f32(a, b): return _binary("dwo_add_f32", a, b, np.float32)
def add_fp16(a, b): return _binary("dwo_add_fp16", a, b, np.uint16)
def mul_f32(a, b): return _binary("dwo_mul_f32", a, b, np.float32)
def mul_fp16(a, b): return _binary("dwo_mul_fp16", a, b, np.uint16)


def silu_fp16(x):
    """Sigmoid then Mul, each rounded to f16 (runtime.rs:1641-1734)."""
    return mul_fp16(x, sigmoid_fp16(x))


def silu_f32(x):
    return mul_f32(x, sigmoid_f32(x))


def requantize_i32_to_i8(x, s):
    x = np.ascontiguousarray(x, np.int32)
    y = np.empty(x.shape, np.int8)
    lib().dwo_requantize_i32_to_i8(_p(y), _p(x), x.size, float(s))
    return y


def quantize_f32_to_i8(x, s):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.int8)
    lib().dwo_quantize_f32_to_i8(_p(y), _p(x), x.size, float(s))
    return y


def dequantize_i8_to_f32(x, s):
    x = np.ascontiguousarray(x, np.int8)
    y = np.empty(x.shape, np.float32)
    lib().dwo_dequantize_i8_to_f32(_p(y), _p(x), x.size, float(s))
    return y


def add_i8(a, b, sa, sb):
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    y = np.empty(a.shape, np.int8)
    lib().dwo_add_i8(_p(y), _p(a), _p(b), a.size, float(sa), float(sb))
    return y


def scale_from_range(mn, mx):
    return float(lib().dwo_scale_from_range(float(mn), float(mx)))


def quantize_weights_per_channel(w_rows):
    """PerChannelScale::from_weights + quantize_weights_per_channel over rows (one row per channel)."""
    w = np.ascontiguousarray(w_rows, np.float32)
    c = w.shape[0]
    q = np.empty(w.shape, np.int8)
    s = np.empty(c, np.float32)
    lib().dwo_quantize_weights_per_channel(_p(q), _p(s), _p(w), c, w.size // c)
    return q, s


def maxpool2d_f32(x, k, s):
    x = np.ascontiguousarray(x, np.float32)
    n, h, w, c = x.shape
    ho, wo = (h - k[0]) // s[0] + 1, (w - k[1]) // s[1] + 1
    y = np.empty((n, ho, wo, c), np.float32)
    lib().dwo_maxpool2d_f32_nhwc(_p(y), _p(x), n, h, w, c, k[0], k[1], s[0], s[1])
    return y


def maxpool2d_padded(x, k, s, pads):
    """pads = (top, left, bottom, right); dtype float32 / uint16 (f16 bits) /
    uint8 / int8 (int8 through the order-preserving map q ^ 0x80 to uint8)."""
    if np.asarray(x).dtype == np.int8:
        u = np.ascontiguousarray(x).view(np.uint8) ^ np.uint8(0x80)
        return (maxpool2d_padded(u, k, s, pads) ^ np.uint8(0x80)).view(np.int8)
    x = np.ascontiguousarray(x)
    n, h, w, c = x.shape
    pt, pl, pb, pr = pads
    ho, wo = (h + pt + pb - k[0]) // s[0] + 1, (w + pl + pr - k[1]) // s[1] + 1
    y = np.empty((n, ho, wo, c), x.dtype)
    lib().dwo_maxpool2d_padded_nhwc(_p(y), _p(x), n, h, w, c, k[0], k[1], s[0], s[1], pt, pl, pb, pr,
                                    x.dtype.itemsize)
    return y


def resize_nearest(x, ho, wo):
    x = np.ascontiguousarray(x)
    n, h, w, c = x.shape
    y = np.empty((n, ho, wo, c), x.dtype)
    lib().dwo_resize_nearest_nhwc(_p(y), _p(x), n, h, w, ho, wo, c, x.dtype.itemsize)
    return y


def concat_channels(xs):
    xs = [np.ascontiguousarray(a) for a in xs]
    pix = xs[0].size // xs[0].shape[-1]
    chans = (C.c_size_t * len(xs))(*[a.shape[-1] for a in xs])
    ptrs = (C.c_void_p * len(xs))(*[_p(a) for a in xs])
    y = np.empty(xs[0].shape[:-1] + (sum(a.shape[-1] for a in xs),), xs[0].dtype)
    lib().dwo_concat_channels(_p(y), ptrs, chans, len(xs), pix, xs[0].dtype.itemsize)
    return y


def split_channels(x, sizes):
    x = np.ascontiguousarray(x)
    pix = x.size // x.shape[-1]
    outs = [np.empty(x.shape[:-1] + (s,), x.dtype) for s in sizes]
    chans = (C.c_size_t * len(sizes))(*sizes)
    ptrs = (C.c_void_p * len(sizes))(*[_p(a) for a in outs])
    lib().dwo_split_channels(ptrs, _p(x), chans, len(sizes), pix, x.dtype.itemsize)
    return outs


def fold_batchnorm(w_oihw, bias, gamma, beta, mean, var, eps):
    """fold_batchnorm arithmetic (graph.rs:597-613); returns (w', b')."""
    w = np.ascontiguousarray(w_oihw, np.float32).copy()
    c = w.shape[0]
    b_out = np.empty(c, np.float32)
    bp = 0
    if bias is not None:
        bias = np.ascontiguousarray(bias, np.float32)
        bp = _p(bias)
    arrs = [np.ascontiguousarray(a, np.float32) for a in (gamma, beta, mean, var)]
    lib().dwo_fold_batchnorm(_p(w), _p(b_out), bp, *[_p(a) for a in arrs], float(eps), c, w.size // c)
    return w, b_out


# --- quantized extensions ----------------------------------------------------
def quantize_linear_f16_u8(xh, scale, zp):
    xh = np.ascontiguousarray(xh, np.uint16)
    y = np.empty(xh.shape, np.uint8)
    lib().dwo_quantize_linear_f16_u8(_p(y), _p(xh), xh.size, float(scale), int(zp))
    return y


def dequantize_linear_u8_f16(x, scale, zp):
    x = np.ascontiguousarray(x, np.uint8)
    y = np.empty(x.shape, np.uint16)
    lib().dwo_dequantize_linear_u8_f16(_p(y), _p(x), x.size, float(scale), int(zp))
    return y


def qlinear_add_u8(a, b, sa, za, sb, zb, sy, zy):
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.uint8)
    y = np.empty(a.shape, np.uint8)
    lib().dwo_qlinear_add_u8(_p(y), _p(a), _p(b), a.size, float(sa), int(za), float(sb), int(zb),
                             float(sy), int(zy))
    return y


def silu_lut_u8(sx, zx, sy, zy):
    lut = np.empty(256, np.uint8)
    lib().dwo_silu_lut_u8(_p(lut), float(sx), int(zx), float(sy), int(zy))
    return lut


def lut_u8(x, lut):
    x = np.ascontiguousarray(x, np.uint8)
    lut = np.ascontiguousarray(lut, np.uint8)
    y = np.empty(x.shape, np.uint8)
    lib().dwo_lut_u8(_p(y), _p(x), x.size, _p(lut))
    return y


# --------------------------------------------------------------------------
# Classifier-head ops (ops.rs:273-290, :461-479, :2981-2995, :1609-1638;
# onnx runtime.rs:1109-1175)
# --------------------------------------------------------------------------
def gemm_f32(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    (m, k), (k2, n) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().dwo_gemm_f32(_p(c), _p(a), _p(b), m, n, k)
    return c


def gemm_fp16(a, b):
    """f16 bit patterns (uint16) in and out."""
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    (m, k), (k2, n) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), np.uint16)
    lib().dwo_gemm_fp16(_p(c), _p(a), _p(b), m, n, k)
    return c


def gemm_i8(a, b):
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.int8)
    (m, k), (k2, n) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), np.int32)
    lib().dwo_gemm_i8(_p(c), _p(a), _p(b), m, n, k)
    return c


def global_avg_pool_f32(x):
    x = np.ascontiguousarray(x, np.float32)
    n, h, w, c = x.shape
    y = np.empty((n, c), np.float32)
    lib().dwo_global_avg_pool_f32(_p(y), _p(x), n, h, w, c)
    return y


def global_avg_pool_fp16(x):
    x = np.ascontiguousarray(x, np.uint16)
    n, h, w, c = x.shape
    y = np.empty((n, c), np.uint16)
    lib().dwo_global_avg_pool_fp16(_p(y), _p(x), n, h, w, c)
    return y


def clip(x, lo, hi):
    """dispatch_clip (onnx runtime.rs:1004-1042): f32::clamp(min, max) (NaN
    passes through); f16 bits through F16::to_f32, clamp, F16::from_f32."""
    if x.dtype == np.uint16:
        return f16_from_f32(clip(f16_to_f32(x), lo, hi))
    x = np.asarray(x, np.float32)
    lo, hi = np.float32(lo), np.float32(hi)
    return np.where(x < lo, lo, np.where(x > hi, hi, x)).astype(np.float32)


def softmax_f16(xh):
    """CpuGraphRuntime::dispatch_softmax for F16 (runtime.rs:1311-1322): every
    input through F16::to_f32, softmax_f32, each output F16::from_f32."""
    return f16_from_f32(softmax_f32(f16_to_f32(xh)))


def softmax_f32(x):
    """Softmax over the last axis."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().dwo_softmax_f32(_p(y), _p(x), x.size // n, n)
    return y


def gemm_tb(a, b):
    """The graph runtime's transposed Gemm: B is [n][k]; f32 or f16 bits
    (uint16) by a's dtype; unfused multiply and add."""
    f16 = a.dtype == np.uint16
    dt = np.uint16 if f16 else np.float32
    a = np.ascontiguousarray(a, dt)
    b = np.ascontiguousarray(b, dt)
    (m, k), (n, k2) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), dt)
    (lib().dwo_gemm_fp16_tb if f16 else lib().dwo_gemm_f32_tb)(_p(c), _p(a), _p(b), m, n, k)
    return c


# --- YOLOv8 detect tail and post-processing (Part C) -----------------------

DETECTION = np.dtype([("bbox", np.float32, 4), ("class_id", np.uint32), ("confidence", np.float32)])


def yolo_detect_tail_f16(levels, strides, nc=80, reg_max=16):
    """The exported detect tail (DFL softmax + 1x1 expectation, dist2bbox,
    sigmoid, concat) over per-level NHWC f16 head outputs [n, h, w, 4*reg_max + nc]
    (uint16 bits).  Returns [n, 4 + nc, A] f32."""
    xs = [np.ascontiguousarray(x, np.uint16) for x in levels]
    n = xs[0].shape[0]
    hs = np.array([x.shape[1] for x in xs], np.int32)
    ws = np.array([x.shape[2] for x in xs], np.int32)
    for x in xs:
        assert x.shape[0] == n and x.shape[3] == 4 * reg_max + nc
    st = np.asarray(strides, np.float32)
    ptrs = (C.c_void_p * len(xs))(*[x.ctypes.data for x in xs])
    A = int((hs * ws).sum())
    out = np.empty((n, 4 + nc, A), np.float32)
    lib().dwo_yolo_detect_tail_f16(_p(out), C.cast(ptrs, C.c_void_p), _p(hs), _p(ws), _p(st), len(xs), n, nc,
                                   reg_max)
    return out


def iou(a, b):
    """iou (postprocess.rs:36-55) of two [x1, y1, x2, y2] boxes."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return float(lib().dwo_iou(_p(a), _p(b)))


def yolo_postprocess(raw, img_w=640, img_h=640, conf=0.25, iou_thr=0.45, agnostic=False):
    """postprocess_yolo (postprocess.rs:279-305) per image of raw [n, 4 + nc, A]
    f32: a list (one per image) of DETECTION arrays in the reference's order."""
    raw = np.ascontiguousarray(raw, np.float32)
    if raw.ndim == 2:
        raw = raw[None]
    n, ch, A = raw.shape
    cap = A
    out = np.zeros((n, cap), DETECTION)
    counts = np.zeros(n, np.uint64)
    lib().dwo_yolo_postprocess(out.ctypes.data, counts.ctypes.data, _p(raw), n, ch - 4, A, img_w, img_h, conf,
                               iou_thr, int(agnostic), cap)
    return [out[b, :int(counts[b])].copy() for b in range(n)]


# --- quantized classifier head ----------------------------------------------

def qgemm_u8s8(a, b, bias, a_scale, a_zp, b_scales, y_scale, y_zp, trans_b=False):
    """QGemm u8 x s8 -> u8: the QLinearConv restatement on a 1x1 kernel over
    the rows of A ([m][k]); B [k][n] (or [n][k] with trans_b)."""
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.int8)
    if trans_b:
        b = np.ascontiguousarray(b.T)
    m, k = a.shape
    n = b.shape[1]
    y = qlinearconv_u8s8(a.reshape(m, 1, 1, k), b.reshape(1, 1, k, n), bias, (1, 1), (0, 0), a_scale, a_zp,
                         b_scales, y_scale, y_zp)
    return y.reshape(m, n)


def qlinear_gap_u8(x, x_scale, x_zp, y_scale, y_zp):
    """QLinearGlobalAveragePool over NHWC u8 [n, h, w, c] -> [n, c]."""
    x = np.ascontiguousarray(x, np.uint8)
    n, h, w, c = x.shape
    y = np.empty((n, c), np.uint8)
    lib().dwo_qlinear_gap_u8(_p(y), _p(x), n, h, w, c, x_scale, x_zp, y_scale, y_zp)
    return y


# --- Part D: layout ops, broadcasting, average pool (numpy restatements) -----

def _f16_round_trip(y):
    """F16::from_f32(to_f32(v)): the identity except subnormals (halved by
    the decode) and NaN payloads (dtype.rs:164-263)."""
    return f16_from_f32(f16_to_f32(y))


def transpose(x, perm, f16_round_trip=True):
    """transpose_f32 (crates/dragonwing-cpu/src/ops.rs:2468-2520) on a tensor
    of rank <= 4 stored row-major: output axis k is input axis perm[k].  An
    f16 tensor goes through to_f32 / from_f32 (dispatch_transpose,
    crates/dragonwing-onnx/src/runtime.rs:2073-2084) unless the transpose is
    a pure layout change (f16_round_trip False)."""
    y = np.ascontiguousarray(np.transpose(np.asarray(x), perm))
    return _f16_round_trip(y) if f16_round_trip and y.dtype == np.uint16 else y


def slice_axes(x, slices, f16_round_trip=True):
    """slice_f32 (ops.rs:2532-2570) with resolved (axis, start, end, step)
    entries (0 <= start <= end <= dim, step >= 1); f16 through f32 as
    dispatch_slice does (runtime.rs:2130-2140)."""
    idx = [slice(None)] * np.asarray(x).ndim
    for ax, st, en, sp in slices:
        idx[ax] = slice(st, en, sp)
    y = np.ascontiguousarray(np.asarray(x)[tuple(idx)])
    return _f16_round_trip(y) if f16_round_trip and y.dtype == np.uint16 else y


_BIN = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide}


def binary(op, a, b):
    """Add / Sub / Mul / Div: one f32 operation per element (add_f32 ops.rs:363-384,
    sub_f32 :1978-2003, mul_f32 :1899-1919, div_f32 :2057-2082); f16
    operands widened with to_f32 and the result stored with from_f32
    (add_fp16 :434-442, sub_fp16 :2038-2046, mul_fp16 :1959-1967,
    div_fp16 :2117-2125).  Broadcasting: the runtime's b[i % len(b)] loops
    (runtime.rs:1045-1860) for a second operand that tiles the first are
    numpy's trailing broadcast; a smaller first operand broadcasts the same
    way (ONNX multidirectional broadcasting)."""
    a, b = np.asarray(a), np.asarray(b)
    f16 = a.dtype == np.uint16
    af = f16_to_f32(a) if f16 else a.astype(np.float32)
    bf = f16_to_f32(b) if f16 else b.astype(np.float32)
    with np.errstate(all="ignore"):
        r = _BIN[op](af, bf, dtype=np.float32)
    return f16_from_f32(r) if f16 else np.ascontiguousarray(r, np.float32)


def avgpool2d_nhwc(x, k, s):
    """avgpool2d_f32_nhwc (ops.rs:1556-1595): unpadded windows, the sum over
    ph then pw in f32, then one division by kh * kw; f16 tensors widened
    with to_f32 and the average stored with from_f32 (runtime.rs:1571-1630)."""
    x = np.asarray(x)
    f16 = x.dtype == np.uint16
    xf = f16_to_f32(x) if f16 else x.astype(np.float32)
    n, h, w, c = xf.shape
    (kh, kw), (sh, sw) = k, s
    ho, wo = (h - kh) // sh + 1, (w - kw) // sw + 1
    acc = np.zeros((n, ho, wo, c), np.float32)
    for ph in range(kh):
        for pw in range(kw):
            acc = (acc + xf[:, ph:ph + (ho - 1) * sh + 1:sh, pw:pw + (wo - 1) * sw + 1:sw, :]).astype(np.float32)
    r = (acc / np.float32(kh * kw)).astype(np.float32)
    return f16_from_f32(r) if f16 else r
