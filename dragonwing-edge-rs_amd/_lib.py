"""ctypes binding of libdwhip.so (the C ABI declared in include/dw_hip.h).

The library is the only compute path: if it is missing or fails to load,
every entry point raises; there is no CPU fallback.
"""
from __future__ import annotations

import atexit
import ctypes as C
import re
import sys
import weakref
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIBPATH = PKG / "libdwhip.so"
HEADER = ROOT / "include" / "dw_hip.h"

P = C.c_void_p
Z = C.c_size_t
F = C.c_float
I = C.c_int
S = C.c_char_p
PP = C.POINTER(C.c_void_p)


class DwOpParams(C.Structure):
    """dw_op_params (include/dw_hip.h): the C form of OpParams."""
    _fields_ = [
        ("kind", I),
        ("kernel_shape", I * 2),
        ("strides", I * 2),
        ("pads", I * 4),
        ("dilations", I * 2),
        ("group", I),
        ("axis", I),
        ("split_sizes", I * 8),
        ("num_splits", I),
        ("out_h", I),
        ("out_w", I),
        ("mode_nearest", I),
        ("scale", F),
        ("scale_a_over_out", F),
        ("scale_b_over_out", F),
        ("has_relu", I),
        ("epsilon", F),
        ("act", I),
        ("alpha", F),
        ("beta", F),
        ("trans_a", I),
        ("trans_b", I),
        ("clip_min", F),
        ("clip_max", F),
        ("reg_max", I),
        ("level_strides", F * 4),
        ("perm", I * 4),
        ("num_slice_axes", I),
        ("slice_axes", I * 4),
        ("slice_starts", I * 4),
        ("slice_ends", I * 4),
        ("slice_steps", I * 4),
    ]


_CONV = [P, P, P, P] + [Z] * 11
SIGNATURES = {
    "dw_last_error": (S, []),
    "dw_hip_backend_create": (I, [I, PP]),
    "dw_hip_backend_destroy": (None, [P]),
    "dw_hip_backend_name": (S, [P]),
    "dw_hip_alloc": (I, [P, Z, I, PP]),
    "dw_hip_buffer_free": (None, [P]),
    "dw_hip_buffer_len_bytes": (Z, [P]),
    "dw_hip_buffer_device_ptr": (P, [P]),
    "dw_hip_upload": (I, [P, P, P, Z]),
    "dw_hip_download": (I, [P, P, P, Z]),
    "dw_hip_synchronize": (I, [P]),
    "dw_hip_conv2d_f32_nhwc": (I, _CONV),
    "dw_hip_conv2d_bias_act_f32_nhwc": (I, [P, P, P, P, P] + [Z] * 11 + [I]),
    "dw_hip_conv2d_bias_act_f16_nhwc": (I, [P, P, P, P, P] + [Z] * 11 + [I, I]),
    "dw_hip_depthwise_conv2d_f16_nhwc": (I, [P, P, P, P, P] + [Z] * 10 + [I]),
    "dw_hip_depthwise_conv2d_f32_nhwc": (I, [P, P, P, P, P] + [Z] * 10 + [I]),
    "dw_hip_qlinearconv_u8s8": (I, [P, P, P, P, P] + [Z] * 11 + [F, I, P, F, I]),
    "dw_hip_qlinearconv_u8s8_noalloc": (I, [P, P, P, P, P] + [Z] * 11 + [F, I, P, F, I]),
    "dw_hip_conv2d_i8_nhwc": (I, _CONV),
    "dw_hip_conv2d_requant_relu_i8": (I, _CONV + [F, I]),
    "dw_hip_relu_f32": (I, [P, P, P, Z]),
    "dw_hip_relu_fp16": (I, [P, P, P, Z]),
    "dw_hip_add_f32": (I, [P, P, P, P, Z]),
    "dw_hip_add_fp16": (I, [P, P, P, P, Z]),
    "dw_hip_mul_f32": (I, [P, P, P, P, Z]),
    "dw_hip_mul_fp16": (I, [P, P, P, P, Z]),
    "dw_hip_sigmoid_f32": (I, [P, P, P, Z]),
    "dw_hip_sigmoid_fp16": (I, [P, P, P, Z]),
    "dw_hip_silu_f32": (I, [P, P, P, Z]),
    "dw_hip_silu_fp16": (I, [P, P, P, Z]),
    "dw_hip_bias_add_f32_nhwc": (I, [P, P, P, Z, Z]),
    "dw_hip_requantize_i32_to_i8": (I, [P, P, P, Z, F]),
    "dw_hip_quantize_f32_to_i8": (I, [P, P, P, Z, F]),
    "dw_hip_dequantize_i8_to_f32": (I, [P, P, P, Z, F]),
    "dw_hip_add_i8": (I, [P, P, P, P, Z, F, F]),
    "dw_hip_relu_i8": (I, [P, P, P, Z]),
    "dw_hip_quantize_linear_f16_u8": (I, [P, P, P, Z, F, I]),
    "dw_hip_dequantize_linear_u8_f16": (I, [P, P, P, Z, F, I]),
    "dw_hip_qlinear_add_u8": (I, [P, P, P, P, Z, F, I, F, I, F, I]),
    "dw_hip_lut_u8": (I, [P, P, P, Z, P]),
    "dw_hip_maxpool2d_nhwc": (I, [P, I, P, P] + [Z] * 12),
    "dw_hip_resize_nearest_nhwc": (I, [P, I, P, P] + [Z] * 6),
    "dw_hip_concat_channels_nhwc": (I, [P, I, PP, P, Z, P, Z]),
    "dw_hip_split_channels_nhwc": (I, [P, I, P, PP, P, Z, Z]),
    "dw_hip_gemm_f32": (I, [P, P, P, P, Z, Z, Z]),
    "dw_hip_gemm_fp16": (I, [P, P, P, P, Z, Z, Z]),
    "dw_hip_gemm_i8": (I, [P, P, P, P, Z, Z, Z]),
    "dw_hip_global_avg_pool_nhwc": (I, [P, I, P, P, Z, Z, Z, Z]),
    "dw_hip_softmax_f32": (I, [P, P, P, Z, Z]),
    "dw_hip_yolo_detect_tail": (I, [P, I, P, P, P, P, I, Z, I, I, P]),
    "dw_graph_from_onnx": (I, [P, Z, P]),
    "dw_onnx_inspect": (I, [P, Z, P, Z, P]),
    "dw_hip_graph_set_input_nchw_f32": (I, [P, C.c_char_p, P, Z]),
    "dw_hip_graph_bind_input_nchw_f32": (I, [P, C.c_char_p, P]),
    "dw_hip_transpose_nchw_to_nhwc": (I, [P, P, P, Z, Z, Z, Z, I]),
    "dw_hip_transpose_nhwc_to_nchw": (I, [P, P, P, Z, Z, Z, Z, I]),
    "dw_hip_fold_batchnorm": (I, [P, P, P, P, P, P, P, C.c_float, Z, Z, P, P]),
    "dw_hip_qgemm_u8s8": (I, [P, P, P, P, P, Z, Z, Z, I, C.c_float, I, P, C.c_float, I]),
    "dw_hip_qlinear_global_avg_pool_u8": (I, [P, P, P, Z, Z, Z, Z, C.c_float, I, C.c_float, I]),
    "dw_hip_yolo_postprocess": (I, [P, P, Z, I, Z, C.c_uint32, C.c_uint32, C.c_float, C.c_float, I, P, Z, P]),
    "dw_graph_create": (I, [I, PP]),
    "dw_graph_destroy": (None, [P]),
    "dw_graph_add_tensor": (I, [P, S, P, I, I]),
    "dw_graph_set_initializer": (I, [P, S, P, Z]),
    "dw_graph_set_quant": (I, [P, S, F, I]),
    "dw_graph_set_channel_scales": (I, [P, S, P, Z]),
    "dw_graph_add_op": (I, [P, S, S, P, I, P, I, C.POINTER(DwOpParams)]),
    "dw_graph_set_io": (I, [P, P, I, P, I]),
    "dw_graph_fold_batchnorm": (I, [P]),
    "dw_graph_convert_nchw_to_nhwc": (I, [P]),
    "dw_graph_apply_fusion_passes": (I, [P, C.POINTER(I)]),
    "dw_op_params_size": (Z, []),
    "dw_graph_convert_to_f16": (I, [P]),
    "dw_graph_set_activation_range": (I, [P, S, F, F]),
    "dw_graph_quantize_qdq": (I, [P, P, I]),
    "dw_hip_calibrate": (I, [P, P, S, P, Z, I]),
    "dw_graph_to_json": (S, [P]),
    "dw_graph_get_initializer": (I, [P, S, PP, C.POINTER(Z)]),
    "dw_hip_graph_runtime_create": (I, [P, P, PP]),
    "dw_hip_graph_runtime_create_ex": (I, [P, P, C.c_uint, PP]),
    "dw_hip_graph_runtime_destroy": (None, [P]),
    "dw_hip_graph_set_input_f32": (I, [P, S, P, Z]),
    "dw_hip_graph_set_input_bytes": (I, [P, S, P, Z]),
    "dw_hip_graph_run": (I, [P]),
    "dw_hip_graph_get_output_f32": (I, [P, S, P, Z]),
    "dw_hip_graph_get_output_bytes": (I, [P, S, P, Z]),
    "dw_hip_graph_tensor_bytes": (I, [P, S, C.POINTER(Z)]),
    "dw_hip_graph_activation_bytes": (I, [P, C.POINTER(Z), C.POINTER(Z)]),
    "dw_hip_graph_enable_capture": (I, [P, I]),
    "dw_hip_graph_num_launches": (I, [P]),
    "dw_hip_graph_launch_info": (S, [P, I]),
    "dw_hip_graph_run_profiled": (I, [P, P]),
    "dw_hip_graph_time_launches": (I, [P, I, P]),
    "dw_hip_graph_time_launches_rotated": (I, [P, I, I, P]),
    "dw_hip_graph_run_unbatched": (I, [P]),
    "dw_hip_graph_num_io": (I, [P, I]),
    "dw_hip_graph_io_name": (S, [P, I, I]),
    "dw_hip_graph_tensor_shape": (I, [P, S, P, P]),
}

_lib = None

# Live native handles, released in this order at interpreter exit: graph
# runtimes (streams, events, captured graphs, device memory), then buffers,
# then backends, then host-only graph IRs.  Objects left to the garbage
# collector during interpreter finalization would otherwise be destroyed in
# whatever order it reaches them, possibly after modules they need are torn
# down; at exit they are released here instead, while the HIP runtime is
# fully up, and their finalizers do nothing afterwards.
RELEASE_RUNTIME, RELEASE_BUFFER, RELEASE_BACKEND, RELEASE_GRAPH = 0, 1, 2, 3
_live = {k: weakref.WeakSet() for k in (RELEASE_RUNTIME, RELEASE_BUFFER, RELEASE_BACKEND, RELEASE_GRAPH)}
_released = False


def track(obj, order: int) -> None:
    """Registers an object with a ``_release()`` method for ordered teardown."""
    _live[order].add(obj)


def native_calls_allowed() -> bool:
    """False once the exit hook has run or the interpreter is finalizing."""
    return not _released and not sys.is_finalizing()


@atexit.register
def release_all() -> None:
    """Releases every live handle (runtimes, buffers, backends, graphs)."""
    global _released
    if _released:
        return
    for order in sorted(_live):
        for obj in list(_live[order]):
            try:
                obj._release()
            except Exception:
                pass
    _released = True


class HipError(RuntimeError):
    """A failing dw_* call: `code` is the dw_status, the message is dw_last_error()."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def header_symbols() -> list[str]:
    """Function names declared in include/dw_hip.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(dw_[a-z0-9_]+)\s*\(", text, re.M)
    return sorted(set(names))


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIBPATH.exists():
            raise RuntimeError(f"{LIBPATH} is not built: run __graft_entry__.build()")
        lib = C.CDLL(str(LIBPATH))
        for name, (res, args) in SIGNATURES.items():
            if not hasattr(lib, name):
                continue  # reported by missing_exports()
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().dw_last_error()
        raise HipError(rc, msg.decode() if msg else "")


def missing_exports() -> list[str]:
    """Header-declared functions the built library does not export."""
    lib = C.CDLL(str(LIBPATH))
    return [n for n in header_symbols() if not hasattr(lib, n)]
