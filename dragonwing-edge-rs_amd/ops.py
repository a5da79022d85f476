"""Op functions: ``dragonwing_vulkan::ops`` signatures on the HIP backend.

Each function takes the backend, device buffers and the reference's scalar
arguments (``crates/dragonwing-vulkan/src/ops.rs``), validates sizes in the
library and enqueues work on the backend stream.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, load

ACT_NONE, ACT_RELU, ACT_SILU = 0, 1, 2
DTYPE_F32, DTYPE_F16, DTYPE_I8, DTYPE_U8, DTYPE_I32 = 0, 1, 2, 3, 4


def _h(b):
    return None if b is None else b.handle


def conv2d_f32_nhwc(be, inp, kernel, out, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w,
                    pad_h, pad_w):
    """vulkan ops.rs:1308 / cpu ops.rs:1356."""
    check(load().dw_hip_conv2d_f32_nhwc(be.handle, inp.handle, kernel.handle, out.handle, n, h_in,
                                        w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w))


def conv2d_bias_act_f32_nhwc(be, inp, kernel, bias, out, n, h_in, w_in, c_in, c_out, k_h, k_w,
                             stride_h, stride_w, pad_h, pad_w, act=ACT_NONE):
    check(load().dw_hip_conv2d_bias_act_f32_nhwc(be.handle, inp.handle, kernel.handle, _h(bias),
                                                 out.handle, n, h_in, w_in, c_in, c_out, k_h, k_w,
                                                 stride_h, stride_w, pad_h, pad_w, act))


def conv2d_bias_act_f16_nhwc(be, inp, kernel, bias, out, n, h_in, w_in, c_in, c_out, k_h, k_w,
                             stride_h, stride_w, pad_h, pad_w, act=ACT_NONE, exact=False):
    check(load().dw_hip_conv2d_bias_act_f16_nhwc(be.handle, inp.handle, kernel.handle, _h(bias),
                                                 out.handle, n, h_in, w_in, c_in, c_out, k_h, k_w,
                                                 stride_h, stride_w, pad_h, pad_w, act, int(exact)))


def depthwise_conv2d_f16_nhwc(be, inp, kernel, bias, out, n, h_in, w_in, c, k_h, k_w, stride_h,
                              stride_w, pad_h, pad_w, act=ACT_NONE):
    check(load().dw_hip_depthwise_conv2d_f16_nhwc(be.handle, inp.handle, kernel.handle, _h(bias),
                                                  out.handle, n, h_in, w_in, c, k_h, k_w, stride_h,
                                                  stride_w, pad_h, pad_w, act))


def depthwise_conv2d_f32_nhwc(be, inp, kernel, bias, out, n, h_in, w_in, c, k_h, k_w, stride_h,
                              stride_w, pad_h, pad_w, act=ACT_NONE):
    check(load().dw_hip_depthwise_conv2d_f32_nhwc(be.handle, inp.handle, kernel.handle, _h(bias),
                                                  out.handle, n, h_in, w_in, c, k_h, k_w, stride_h,
                                                  stride_w, pad_h, pad_w, act))


def qlinearconv_u8s8(be, inp, kernel, bias, out, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h,
                     stride_w, pad_h, pad_w, x_scale, x_zp, w_scales, y_scale, y_zp):
    ws = np.ascontiguousarray(w_scales, np.float32)
    assert ws.size == c_out
    check(load().dw_hip_qlinearconv_u8s8(be.handle, inp.handle, kernel.handle, _h(bias), out.handle, n,
                                         h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h,
                                         pad_w, float(x_scale), int(x_zp), ws.ctypes.data,
                                         float(y_scale), int(y_zp)))


def qlinearconv_u8s8_noalloc(be, inp, kernel, bias, out, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h,
                             stride_w, pad_h, pad_w, x_scale, x_zp, w_scales, y_scale, y_zp):
    """qlinearconv_u8s8 with no device allocation (the per-device scratch)."""
    ws = np.ascontiguousarray(w_scales, np.float32)
    assert ws.size == c_out
    check(load().dw_hip_qlinearconv_u8s8_noalloc(be.handle, inp.handle, kernel.handle, _h(bias), out.handle, n,
                                                 h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h,
                                                 pad_w, float(x_scale), int(x_zp), ws.ctypes.data,
                                                 float(y_scale), int(y_zp)))


def conv2d_i8_nhwc(be, inp, kernel, out_i32, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h,
                   stride_w, pad_h, pad_w):
    check(load().dw_hip_conv2d_i8_nhwc(be.handle, inp.handle, kernel.handle, out_i32.handle, n, h_in,
                                       w_in, c_in, c_out, k_h, k_w, stride_h, stride_w, pad_h, pad_w))


def conv2d_requant_relu_i8(be, inp, kernel, out, n, h_in, w_in, c_in, c_out, k_h, k_w, stride_h,
                           stride_w, pad_h, pad_w, requant_scale, do_relu):
    """vulkan ops.rs:2294 conv2d_requant_relu_i8_packed."""
    check(load().dw_hip_conv2d_requant_relu_i8(be.handle, inp.handle, kernel.handle, out.handle, n,
                                               h_in, w_in, c_in, c_out, k_h, k_w, stride_h, stride_w,
                                               pad_h, pad_w, float(requant_scale), int(do_relu)))


def _u(name):
    def f(be, x, y, count):
        check(getattr(load(), name)(be.handle, x.handle, y.handle, count))
    f.__name__ = name
    return f


def _b(name):
    def f(be, a, b, y, count):
        check(getattr(load(), name)(be.handle, a.handle, b.handle, y.handle, count))
    f.__name__ = name
    return f


relu_f32 = _u("dw_hip_relu_f32")
relu_fp16 = _u("dw_hip_relu_fp16")
sigmoid_f32 = _u("dw_hip_sigmoid_f32")
sigmoid_fp16 = _u("dw_hip_sigmoid_fp16")
silu_f32 = _u("dw_hip_silu_f32")
silu_fp16 = _u("dw_hip_silu_fp16")
relu_i8 = _u("dw_hip_relu_i8")
add_f32 = _b("dw_hip_add_f32")
add_fp16 = _b("dw_hip_add_fp16")
mul_f32 = _b("dw_hip_mul_f32")
mul_fp16 = _b("dw_hip_mul_fp16")


def bias_add_f32_nhwc(be, y, bias, count, c):
    check(load().dw_hip_bias_add_f32_nhwc(be.handle, y.handle, bias.handle, count, c))


def requantize_i32_to_i8(be, x, y, count, requant_scale):
    check(load().dw_hip_requantize_i32_to_i8(be.handle, x.handle, y.handle, count, float(requant_scale)))


def quantize_f32_to_i8(be, x, y, count, scale):
    check(load().dw_hip_quantize_f32_to_i8(be.handle, x.handle, y.handle, count, float(scale)))


def dequantize_i8_to_f32(be, x, y, count, scale):
    check(load().dw_hip_dequantize_i8_to_f32(be.handle, x.handle, y.handle, count, float(scale)))


def add_i8(be, a, b, y, count, scale_a_over_y, scale_b_over_y):
    check(load().dw_hip_add_i8(be.handle, a.handle, b.handle, y.handle, count, float(scale_a_over_y),
                               float(scale_b_over_y)))


def quantize_linear_f16_u8(be, x, y, count, scale, zp):
    check(load().dw_hip_quantize_linear_f16_u8(be.handle, x.handle, y.handle, count, float(scale), int(zp)))


def dequantize_linear_u8_f16(be, x, y, count, scale, zp):
    check(load().dw_hip_dequantize_linear_u8_f16(be.handle, x.handle, y.handle, count, float(scale), int(zp)))


def qlinear_add_u8(be, a, b, y, count, a_scale, a_zp, b_scale, b_zp, y_scale, y_zp):
    check(load().dw_hip_qlinear_add_u8(be.handle, a.handle, b.handle, y.handle, count, float(a_scale),
                                       int(a_zp), float(b_scale), int(b_zp), float(y_scale), int(y_zp)))


def lut_u8(be, x, y, count, lut):
    t = np.ascontiguousarray(lut, np.uint8)
    assert t.size == 256
    check(load().dw_hip_lut_u8(be.handle, x.handle, y.handle, count, t.ctypes.data))


def maxpool2d_nhwc(be, dtype, x, y, n, h_in, w_in, c, pool_h, pool_w, stride_h, stride_w,
                   pads=(0, 0, 0, 0)):
    check(load().dw_hip_maxpool2d_nhwc(be.handle, dtype, x.handle, y.handle, n, h_in, w_in, c, pool_h,
                                       pool_w, stride_h, stride_w, *pads))


def resize_nearest_nhwc(be, dtype, x, y, n, h_in, w_in, h_out, w_out, c):
    check(load().dw_hip_resize_nearest_nhwc(be.handle, dtype, x.handle, y.handle, n, h_in, w_in, h_out,
                                            w_out, c))


def concat_channels_nhwc(be, dtype, inputs, channels, y, pixels):
    arr = (C.c_void_p * len(inputs))(*[b.handle for b in inputs])
    ch = (C.c_size_t * len(channels))(*channels)
    check(load().dw_hip_concat_channels_nhwc(be.handle, dtype, arr, ch, len(inputs), y.handle, pixels))


def split_channels_nhwc(be, dtype, x, outputs, channels, pixels):
    arr = (C.c_void_p * len(outputs))(*[b.handle for b in outputs])
    ch = (C.c_size_t * len(channels))(*channels)
    check(load().dw_hip_split_channels_nhwc(be.handle, dtype, x.handle, arr, ch, len(outputs), pixels))


# Classifier-head ops (row-major; see include/dw_hip.h)
def gemm_f32(be, a, b, c, m, n, k):
    check(load().dw_hip_gemm_f32(be.handle, a.handle, b.handle, c.handle, m, n, k))


def gemm_fp16(be, a, b, c, m, n, k):
    check(load().dw_hip_gemm_fp16(be.handle, a.handle, b.handle, c.handle, m, n, k))


def gemm_i8(be, a, b, c_i32, m, n, k):
    check(load().dw_hip_gemm_i8(be.handle, a.handle, b.handle, c_i32.handle, m, n, k))


def global_avg_pool_nhwc(be, dtype, x, y, n, h, w, c):
    check(load().dw_hip_global_avg_pool_nhwc(be.handle, dtype, x.handle, y.handle, n, h, w, c))


def softmax_f32(be, x, y, rows, n):
    check(load().dw_hip_softmax_f32(be.handle, x.handle, y.handle, rows, n))


# --- YOLOv8 detect tail and post-processing ---------------------------------

DETECTION = np.dtype([("bbox", np.float32, 4), ("class_id", np.uint32), ("confidence", np.float32)])


def yolo_detect_tail(be, levels, hw, strides, n, out, nc=80, reg_max=16, dtype=DTYPE_F16):
    """The exported detect tail (DFL, dist2bbox, sigmoid, concat) over the
    per-level NHWC head outputs (buffers of [n, h, w, 4*reg_max + nc]) into
    out [n, 4 + nc, A] f32.  hw: [(h, w)] per level."""
    k = len(levels)
    bufs = (C.c_void_p * k)(*[b.handle for b in levels])
    hs = (C.c_int * k)(*[int(h) for h, _ in hw])
    ws = (C.c_int * k)(*[int(w) for _, w in hw])
    st = (C.c_float * k)(*[float(s) for s in strides])
    check(load().dw_hip_yolo_detect_tail(be.handle, dtype, C.cast(bufs, C.c_void_p), C.cast(hs, C.c_void_p),
                                         C.cast(ws, C.c_void_p), C.cast(st, C.c_void_p), k, n, nc, reg_max,
                                         out.handle))


def yolo_postprocess(be, raw, n, nc, num_det, img_w=640, img_h=640, conf=0.25, iou=0.45, agnostic=False,
                     cap=None):
    """postprocess_yolo (postprocess.rs:279-305) per image of the device
    buffer raw [n, 4 + nc, num_det] f32: a list of DETECTION arrays, one per
    image, in the reference's order."""
    cap = num_det if cap is None else cap
    out = np.zeros((n, cap), DETECTION)
    counts = np.zeros(n, np.uint64)
    check(load().dw_hip_yolo_postprocess(be.handle, raw.handle, n, nc, num_det, img_w, img_h, conf, iou,
                                         int(agnostic), out.ctypes.data, cap, counts.ctypes.data))
    return [out[b, :int(counts[b])].copy() for b in range(n)]


# --- quantized classifier head ------------------------------------------------

def qgemm_u8s8(be, a, b, bias, y, m, n, k, a_scale, a_zp, b_scales, y_scale, y_zp, trans_b=False):
    """QGemm u8 x s8 -> u8 (per-column weight scales, int32 bias, RNE)."""
    sc = np.ascontiguousarray(b_scales, np.float32)
    check(load().dw_hip_qgemm_u8s8(be.handle, a.handle, b.handle, _h(bias), y.handle, m, n, k, int(trans_b),
                                   float(a_scale), int(a_zp), sc.ctypes.data, float(y_scale), int(y_zp)))


def qlinear_global_avg_pool_u8(be, x, y, n, h, w, c, x_scale, x_zp, y_scale, y_zp):
    check(load().dw_hip_qlinear_global_avg_pool_u8(be.handle, x.handle, y.handle, n, h, w, c, float(x_scale),
                                                   int(x_zp), float(y_scale), int(y_zp)))


# --- layout and BN fold on the device -----------------------------------------

def transpose_nchw_to_nhwc(be, x, y, n, c, h, w, dtype=DTYPE_F32):
    """graph.rs:339-356 on the device."""
    check(load().dw_hip_transpose_nchw_to_nhwc(be.handle, x.handle, y.handle, n, c, h, w, dtype))


def transpose_nhwc_to_nchw(be, x, y, n, h, w, c, dtype=DTYPE_F32):
    """graph.rs:358-379 on the device."""
    check(load().dw_hip_transpose_nhwc_to_nchw(be.handle, x.handle, y.handle, n, h, w, c, dtype))


def fold_batchnorm(be, w, bias, gamma, beta, mean, var, eps, c_out, per_channel, w_out, bias_out):
    """fold_batchnorm (graph.rs:521-690) on device buffers (f32, f64 math)."""
    check(load().dw_hip_fold_batchnorm(be.handle, w.handle, _h(bias), gamma.handle, beta.handle, mean.handle,
                                       var.handle, float(eps), c_out, per_channel, w_out.handle, bias_out.handle))
