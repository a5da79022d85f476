"""GPU parity of the classifier-head ops (Gemm f32 / f16 / int8,
GlobalAveragePool, Softmax) against the oracle, through the C ABI.

Bars: bit-exact for Gemm and GlobalAveragePool (the reference's order of
accumulation); Softmax within 1e-5 relative (the device expf and glibc expf
may differ in the last bits)."""
import numpy as np
import pytest

import oracle
import dragonwing_edge_rs_amd as dw
from dragonwing_edge_rs_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mnk", [(32, 1000, 1280), (3, 5, 7), (1, 300, 17)])
def test_gemm_f32_bit_exact(backend, mnk):
    m, n, k = mnk
    r = np.random.default_rng(sum(mnk))
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (k, n)).astype(np.float32)
    ba, bb, bc = backend.from_numpy(a), backend.from_numpy(b), backend.alloc(m * n * 4)
    ops.gemm_f32(backend, ba, bb, bc, m, n, k)
    np.testing.assert_array_equal(backend.to_numpy(bc, np.float32, (m, n)), oracle.gemm_f32(a, b))


@pytest.mark.parametrize("mnk", [(32, 1000, 1280), (2, 70, 9)])
def test_gemm_fp16_bit_exact(backend, mnk):
    m, n, k = mnk
    r = np.random.default_rng(7 + sum(mnk))
    a = r.normal(0, 1, (m, k)).astype(np.float16).view(np.uint16)
    b = r.normal(0, 0.1, (k, n)).astype(np.float16).view(np.uint16)
    a.ravel()[::97] = np.uint16(0x0003)  # subnormal operands: decoded at half value
    b.ravel()[::89] = np.uint16(0x8201)
    ba, bb, bc = backend.from_numpy(a), backend.from_numpy(b), backend.alloc(m * n * 2)
    ops.gemm_fp16(backend, ba, bb, bc, m, n, k)
    np.testing.assert_array_equal(backend.to_numpy(bc, np.uint16, (m, n)), oracle.gemm_fp16(a, b))


def test_gemm_i8_exact(backend):
    m, n, k = 32, 1000, 1280
    r = np.random.default_rng(11)
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    b = r.integers(-128, 128, (k, n)).astype(np.int8)
    ba, bb, bc = backend.from_numpy(a), backend.from_numpy(b), backend.alloc(m * n * 4)
    ops.gemm_i8(backend, ba, bb, bc, m, n, k)
    got = backend.to_numpy(bc, np.int32, (m, n))
    np.testing.assert_array_equal(got, oracle.gemm_i8(a, b))
    np.testing.assert_array_equal(got, a.astype(np.int64) @ b.astype(np.int64))


def test_gemm_rejects_size_mismatch(backend):
    a, b = backend.alloc(3 * 4 * 4), backend.alloc(4 * 5 * 4)
    with pytest.raises(dw.HipError):
        ops.gemm_f32(backend, a, b, backend.alloc(4), 3, 5, 4)


@pytest.mark.parametrize("shape", [(32, 7, 7, 1280), (3, 5, 9, 70)])
def test_global_avg_pool_bit_exact(backend, shape):
    n, h, w, c = shape
    r = np.random.default_rng(sum(shape))
    x = r.normal(0, 2, shape).astype(np.float32)
    bx, by = backend.from_numpy(x), backend.alloc(n * c * 4)
    ops.global_avg_pool_nhwc(backend, ops.DTYPE_F32, bx, by, n, h, w, c)
    np.testing.assert_array_equal(backend.to_numpy(by, np.float32, (n, c)), oracle.global_avg_pool_f32(x))
    xh = x.astype(np.float16).view(np.uint16)
    xh.ravel()[::53] = np.uint16(0x0005)
    bx, by = backend.from_numpy(xh), backend.alloc(n * c * 2)
    ops.global_avg_pool_nhwc(backend, ops.DTYPE_F16, bx, by, n, h, w, c)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, (n, c)), oracle.global_avg_pool_fp16(xh))


@pytest.mark.parametrize("rows_n", [(32, 1000), (25600, 16), (3, 1)])
def test_softmax_f32(backend, rows_n):
    rows, n = rows_n
    x = np.random.default_rng(rows + n).normal(0, 4, (rows, n)).astype(np.float32)
    bx, by = backend.from_numpy(x), backend.alloc(x.nbytes)
    ops.softmax_f32(backend, bx, by, rows, n)
    got = backend.to_numpy(by, np.float32, (rows, n))
    ref = oracle.softmax_f32(x)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30)
    np.testing.assert_allclose(got.astype(np.float64).sum(axis=1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("trans_b", [0, 1])
def test_classifier_head_graph_bit_exact(backend, f16, trans_b):
    # GlobalAveragePool -> Flatten -> Gemm (+ bias), and MatMul, on the graph
    # runtime against the oracle's CpuGraph (dispatch_global_avg_pool,
    # dispatch_reshape, dispatch_gemm: fma chain without transposes, separate
    # multiply and add with trans_b; then the bias pass).
    from dragonwing_edge_rs_amd.graph import Graph, GRAPH_F16, GRAPH_F32, HipGraphRuntime
    from oracle.cpu_graph import CpuGraph
    r = np.random.default_rng(40 + 2 * trans_b + f16)
    n, h, w, c, k = 5, 7, 7, 64, 100
    dt = "f16" if f16 else "f32"
    cast = (lambda a: a.astype(np.float16).view(np.uint16)) if f16 else (lambda a: a.astype(np.float32))
    x = cast(r.normal(0, 1, (n, h, w, c)))
    wt = cast(r.normal(0, 0.1, (k, c) if trans_b else (c, k)))
    b = cast(r.normal(0, 0.1, (k,)))
    w2 = cast(r.normal(0, 0.1, (k, 10)))
    g = Graph(GRAPH_F16 if f16 else GRAPH_F32)
    g.add_tensor("x", x.shape, dt)
    g.add_tensor("pool", (n, 1, 1, c), dt)
    g.add_tensor("flat", (n, c), dt)
    g.add_initializer("w", wt, dt)
    g.add_initializer("b", b, dt)
    g.add_initializer("w2", w2, dt)
    g.add_tensor("logits", (n, k), dt)
    g.add_tensor("out", (n, 10), dt)
    g.add_op("gap", "GlobalAveragePool", ["x"], ["pool"])
    g.add_op("flatten", "Flatten", ["pool"], ["flat"])
    g.add_op("fc", "Gemm", ["flat", "w", "b"], ["logits"], trans_b=trans_b)
    g.add_op("mm", "MatMul", ["logits", "w2"], ["out"])
    g.set_io(["x"], ["logits", "out"])
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", x)
    rt.run()
    cg = CpuGraph(g.to_dict(), g.initializer)
    cg.set_input("x", x)
    ref = cg.run()
    for o, shp in (("logits", (n, k)), ("out", (n, 10))):
        got = rt.get_output_bytes(o).view(np.uint16 if f16 else np.float32).reshape(shp)
        np.testing.assert_array_equal(got, ref[o], err_msg=o)


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("mnk", [(32, 1000, 1280), (5, 12, 48)])
def test_qgemm_u8s8_bit_exact(backend, mnk, trans_b):
    # QGemm on the MFMA implicit-GEMM kernels (1x1 over the rows of A)
    m, n, k = mnk
    r = np.random.default_rng(m + n + k + trans_b)
    a = r.integers(0, 256, (m, k)).astype(np.uint8)
    b = r.integers(-127, 128, (n, k) if trans_b else (k, n)).astype(np.int8)
    bias = r.integers(-4096, 4097, n).astype(np.int32)
    bs = np.exp(r.uniform(np.log(1e-3), np.log(1e-2), n)).astype(np.float32)
    ba, bb, bbias, by = backend.from_numpy(a), backend.from_numpy(b), backend.from_numpy(bias), backend.alloc(m * n)
    ops.qgemm_u8s8(backend, ba, bb, bbias, by, m, n, k, 0.02, 131, bs, 0.05, 120, trans_b=trans_b)
    got = backend.to_numpy(by, np.uint8, (m, n))
    np.testing.assert_array_equal(got, oracle.qgemm_u8s8(a, b, bias, 0.02, 131, bs, 0.05, 120, trans_b=trans_b))


@pytest.mark.parametrize("shape", [(32, 7, 7, 1280), (3, 5, 9, 70)])
def test_qlinear_global_avg_pool_bit_exact(backend, shape):
    r = np.random.default_rng(sum(shape))
    x = r.integers(0, 256, shape).astype(np.uint8)
    n, h, w, c = shape
    bx, by = backend.from_numpy(x), backend.alloc(n * c)
    ops.qlinear_global_avg_pool_u8(backend, bx, by, n, h, w, c, 0.03, 125, 0.01, 128)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint8, (n, c)), oracle.qlinear_gap_u8(x, 0.03, 125, 0.01, 128))


@pytest.mark.parametrize("trans_b", [0, 1])
def test_quantized_classifier_graph_bit_exact(backend, trans_b):
    # A MobileNetV2-style classifier tail (1x1 conv 320 -> 1280 with SiLU,
    # GlobalAveragePool, Flatten, Gemm 1280 -> 1000 with bias), calibrated on
    # the GPU, QDQ-quantized (QLinearConv + table, QLinearGlobalAveragePool,
    # Flatten, QGemm), run on the graph runtime and compared with the
    # oracle's CpuGraph bit for bit.
    from dragonwing_edge_rs_amd.graph import GRAPH_F32, Graph, HipGraphRuntime, calibrate
    from oracle.cpu_graph import CpuGraph
    r = np.random.default_rng(90 + trans_b)
    n = 8

    def build(batch):
        g = Graph(GRAPH_F32)
        g.add_tensor("x", (batch, 7, 7, 320))
        g.add_initializer("cw", r2.uniform(-0.1, 0.1, (1, 1, 320, 1280)).astype(np.float32))
        g.add_initializer("cb", r2.uniform(-0.1, 0.1, 1280).astype(np.float32))
        g.add_tensor("c", (batch, 7, 7, 1280))
        g.add_tensor("s", (batch, 7, 7, 1280))
        g.add_tensor("a", (batch, 7, 7, 1280))
        g.add_tensor("pool", (batch, 1, 1, 1280))
        g.add_tensor("flat", (batch, 1280))
        wshape = (1000, 1280) if trans_b else (1280, 1000)
        g.add_initializer("w", r2.normal(0, 0.03, wshape).astype(np.float32))
        g.add_initializer("b", r2.normal(0, 0.1, 1000).astype(np.float32))
        g.add_tensor("y", (batch, 1000))
        g.add_op("conv", "Conv", ["x", "cw", "cb"], ["c"], kernel_shape=(1, 1))
        g.add_op("sig", "Sigmoid", ["c"], ["s"])
        g.add_op("mul", "Mul", ["c", "s"], ["a"])
        g.add_op("gap", "GlobalAveragePool", ["a"], ["pool"])
        g.add_op("flatten", "Flatten", ["pool"], ["flat"])
        g.add_op("fc", "Gemm", ["flat", "w", "b"], ["y"], trans_b=trans_b)
        g.set_io(["x"], ["y"])
        return g

    r2 = np.random.default_rng(5)
    gc = build(8)
    calib = r.normal(0, 1, (16, 7, 7, 320)).astype(np.float32)
    calibrate(backend, gc, "x", calib)
    ranges = {k: v["range"] for k, v in gc.to_dict()["tensors"].items() if "range" in v}
    r2 = np.random.default_rng(5)
    g = build(n)
    for k, (lo, hi) in ranges.items():
        g.set_activation_range(k, lo, hi)
    g.quantize_qdq()
    types = [op["type"] for op in g.to_dict()["ops"]]
    assert "QGemm" in types and "QLinearGlobalAveragePool" in types, types
    x = r.normal(0, 1, (n, 7, 7, 320)).astype(np.float32)
    xh = oracle.f16_from_f32(x)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", xh)
    rt.run()
    got = rt.get_output_bytes("y").view(np.uint8).reshape(n, 1000)
    cg = CpuGraph(g.to_dict(), g.initializer)
    cg.set_input("x", xh)
    ref = cg.run()["y"]
    np.testing.assert_array_equal(got, ref)
    assert len(np.unique(ref)) > 20  # a spread of levels, not a saturated output
