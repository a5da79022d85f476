"""GPU side of the graph boundary: NCHW <-> NHWC transposes
(transpose_nchw_to_nhwc / transpose_nhwc_to_nchw, onnx graph.rs:339-379),
fold_batchnorm on device weights (graph.rs:521-690, f64 as the oracle), and
graph inputs given in NCHW f32, read by the stem conv's own loader (f16
graphs) or transposed on the device (other graphs).

Bars: transposes move bits (exact); the BN fold is bit-exact against the
oracle; an NCHW input gives exactly the outputs of the same data given in
NHWC through set_input_f32."""
import numpy as np
import pytest

import oracle
from dragonwing_edge_rs_amd import ops, yolo
from dragonwing_edge_rs_amd.graph import HipGraphRuntime

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,npdt", [(ops.DTYPE_F32, np.float32), (ops.DTYPE_F16, np.uint16),
                                        (ops.DTYPE_U8, np.uint8)])
@pytest.mark.parametrize("shape", [(2, 3, 640, 640), (3, 144, 20, 20), (1, 37, 5, 33)])
def test_transposes_round_trip(backend, dtype, npdt, shape):
    r = np.random.default_rng(sum(shape) + dtype)
    n, c, h, w = shape
    x = r.integers(0, np.iinfo(np.uint8).max if npdt == np.uint8 else 60000, shape).astype(npdt)
    if npdt == np.float32:
        x = r.normal(0, 1, shape).astype(np.float32)
    bx, by, bz = backend.from_numpy(x), backend.alloc(x.nbytes), backend.alloc(x.nbytes)
    ops.transpose_nchw_to_nhwc(backend, bx, by, n, c, h, w, dtype)
    y = backend.to_numpy(by, npdt, (n, h, w, c))
    np.testing.assert_array_equal(y, x.transpose(0, 2, 3, 1))
    ops.transpose_nhwc_to_nchw(backend, by, bz, n, h, w, c, dtype)
    np.testing.assert_array_equal(backend.to_numpy(bz, npdt, shape), x)


@pytest.mark.parametrize("with_bias", [False, True])
def test_fold_batchnorm_bit_exact(backend, with_bias):
    r = np.random.default_rng(3 + with_bias)
    co, ci, k = 256, 128, 3
    w = r.uniform(-0.1, 0.1, (co, ci, k, k)).astype(np.float32)
    bias = r.uniform(-0.1, 0.1, co).astype(np.float32) if with_bias else None
    gamma = r.uniform(0.5, 1.5, co).astype(np.float32)
    beta = r.uniform(-0.1, 0.1, co).astype(np.float32)
    mean = r.uniform(-0.1, 0.1, co).astype(np.float32)
    var = r.uniform(0.5, 1.5, co).astype(np.float32)
    var[:4] = (0.0, 1e-30, 3e38, 1e-3)  # edge variances
    bufs = [backend.from_numpy(a) for a in (w, gamma, beta, mean, var)]
    bb = backend.from_numpy(bias) if with_bias else None
    wo, bo = backend.alloc(w.nbytes), backend.alloc(co * 4)
    ops.fold_batchnorm(backend, bufs[0], bb, bufs[1], bufs[2], bufs[3], bufs[4], 1e-3, co, ci * k * k, wo, bo)
    rw, rb = oracle.fold_batchnorm(w, bias, gamma, beta, mean, var, 1e-3)
    np.testing.assert_array_equal(backend.to_numpy(wo, np.float32, w.shape), rw)
    np.testing.assert_array_equal(backend.to_numpy(bo, np.float32, (co,)), rb)


def outputs(rt, info):
    return [rt.get_output_bytes(o).copy() for o in info["outputs"]]


def test_nchw_input_int8_graph_full_workload(backend):
    # the headline graph: the stem reads the NCHW f32 planes itself
    g, info = yolo.int8_graph(backend, batch=32, size=640)
    x = yolo.input_images(32, 640)
    xn = np.ascontiguousarray(x.transpose(0, 3, 1, 2))
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    want = outputs(rt, info)
    rt.set_input_nchw_f32(info["input"], xn)
    rt.run()
    for a, b in zip(outputs(rt, info), want):
        assert a.tobytes() == b.tobytes()
    # a device buffer bound as the input, read by every run
    buf = backend.from_numpy(xn)
    rt.bind_input_nchw_f32(info["input"], buf)
    rt.run()
    for a, b in zip(outputs(rt, info), want):
        assert a.tobytes() == b.tobytes()
    # back to NHWC input: the stem reads the NHWC tensor again
    x2 = yolo.input_images(32, 640, index=7)
    rt.set_input_f32(info["input"], x2)
    rt.run()
    got2 = outputs(rt, info)
    rt.set_input_nchw_f32(info["input"], np.ascontiguousarray(x2.transpose(0, 3, 1, 2)))
    rt.enable_capture(True)
    rt.run()
    rt.run()
    for a, b in zip(outputs(rt, info), got2):
        assert a.tobytes() == b.tobytes()


def test_nchw_input_special_values_f16_graph(backend):
    # values that round to f16 subnormals, overflow to inf, NaN and ties:
    # the stem's loader must round as the host conversion does
    g, info = yolo.f16_graph(batch=2, size=64)
    x = yolo.input_images(2, 64)
    x[0, 0, :8, 0] = [1e-6, -3e-7, 7e4, -1e5, np.nan, 2.0 ** -25, 1 + 2.0 ** -11, 0.0]
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    want = outputs(rt, info)
    rt.set_input_nchw_f32(info["input"], np.ascontiguousarray(x.transpose(0, 3, 1, 2)))
    rt.run()
    for a, b in zip(outputs(rt, info), want):
        assert a.tobytes() == b.tobytes()


def test_nchw_input_f32_graph_by_transpose(backend):
    # an f32 graph: the input is transposed on the device at each run
    g, info = yolo.calibration_graph(1, 64)
    x = yolo.input_images(1, 64)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    want = outputs(rt, info)
    buf = backend.from_numpy(np.ascontiguousarray(x.transpose(0, 3, 1, 2)))
    rt.bind_input_nchw_f32(info["input"], buf)
    rt.run()
    for a, b in zip(outputs(rt, info), want):
        assert a.tobytes() == b.tobytes()
