"""Pins the oracle's classifier-head ops (Gemm f32/f16/int8,
GlobalAveragePool, Softmax) against the reference's known-answer tests
(crates/dragonwing-cpu/src/ops.rs: gemm_i8_scalar_basic :1111-1125,
softmax_basic :765-777, gemm_f32_mt_matches_naive :784-800), closed forms
and float64 evaluations."""
import numpy as np

import oracle


def test_gemm_i8_known_answer():
    # ops.rs:1111-1125: [[1,2,3],[4,5,6]] x [[7,8],[9,10],[11,12]]
    a = np.array([[1, 2, 3], [4, 5, 6]], np.int8)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.int8)
    np.testing.assert_array_equal(oracle.gemm_i8(a, b), [[58, 64], [139, 154]])


def test_gemm_i8_is_the_integer_product():
    r = np.random.default_rng(5)
    a = r.integers(-128, 128, (7, 300), dtype=np.int64)
    b = r.integers(-128, 128, (300, 11), dtype=np.int64)
    np.testing.assert_array_equal(oracle.gemm_i8(a.astype(np.int8), b.astype(np.int8)), a @ b)


def test_gemm_f32_exact_on_integers_and_orientation():
    # small integers: every partial sum is exact, so the result is the
    # integer product; the shapes (3x4)(4x5) catch a transposed operand
    a = np.arange(12, dtype=np.float32).reshape(3, 4) - 5
    b = np.arange(20, dtype=np.float32).reshape(4, 5) * 2 - 7
    np.testing.assert_array_equal(oracle.gemm_f32(a, b), (a.astype(np.int64) @ b.astype(np.int64)))


def test_gemm_f32_reference_inputs_close_to_f64():
    # the inputs of ops.rs:784-800 (sin / cos ramps), 64 x 64 x 64
    m = n = k = 64
    a = np.sin(np.arange(m * k, dtype=np.float32) * np.float32(0.01)).reshape(m, k).astype(np.float32)
    b = np.cos(np.arange(k * n, dtype=np.float32) * np.float32(0.02)).reshape(k, n).astype(np.float32)
    c = oracle.gemm_f32(a, b)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(c - ref)) < 1e-4


def test_gemm_f32_is_a_sequential_fma_chain():
    # a chain whose f32 result depends on the order: 1e8 + 1 - 1e8 ...
    a = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    b = np.ones((4, 1), np.float32)
    # in order: 1e8, 1e8 (the 1 is lost), 0, 1
    assert oracle.gemm_f32(a, b)[0, 0] == 1.0


def test_gemm_fp16_is_f32_chain_of_widened_operands():
    r = np.random.default_rng(9)
    a = r.normal(0, 1, (5, 40)).astype(np.float16).view(np.uint16)
    b = r.normal(0, 1, (40, 6)).astype(np.float16).view(np.uint16)
    c = oracle.gemm_fp16(a, b)
    c32 = oracle.gemm_f32(oracle.f16_to_f32(a).reshape(5, 40), oracle.f16_to_f32(b).reshape(40, 6))
    np.testing.assert_array_equal(c, c32.astype(np.float16).view(np.uint16))


def test_gemm_fp16_subnormal_operand_decoded_at_half():
    # F16::to_f32 returns subnormals at half their IEEE value (dtype.rs:226-263):
    # 0x0002 (2^-23) times 1.0 gives 2^-24 = 0x0001
    a = np.array([[0x0002]], np.uint16)
    b = np.array([[0x3C00]], np.uint16)
    assert int(oracle.gemm_fp16(a, b)[0, 0]) == 0x0001


def test_global_avg_pool_closed_forms():
    x = np.full((2, 7, 7, 5), 0.75, np.float32)
    np.testing.assert_array_equal(oracle.global_avg_pool_f32(x), np.full((2, 5), 0.75, np.float32))
    # integers: exact sum, mean of 0..48 is 24 in every channel
    x = np.broadcast_to(np.arange(49, dtype=np.float32).reshape(1, 7, 7, 1), (3, 7, 7, 4)).copy()
    np.testing.assert_array_equal(oracle.global_avg_pool_f32(x), np.full((3, 4), 24.0, np.float32))
    # channels and batches are not mixed
    r = np.random.default_rng(2)
    x = r.normal(0, 1, (2, 3, 4, 6)).astype(np.float32)
    np.testing.assert_allclose(oracle.global_avg_pool_f32(x), x.astype(np.float64).mean(axis=(1, 2)), rtol=0,
                               atol=1e-6)


def test_global_avg_pool_fp16():
    r = np.random.default_rng(3)
    x = r.normal(0, 1, (2, 5, 5, 8)).astype(np.float16)
    y = oracle.global_avg_pool_fp16(x.view(np.uint16))
    ref = oracle.global_avg_pool_f32(x.astype(np.float32)).astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(y, ref)


def test_softmax_known_answer_and_f64():
    # ops.rs:765-777: [1, 2, 3] sums to 1, positive, order kept
    y = oracle.softmax_f32(np.array([1.0, 2.0, 3.0], np.float32))
    assert abs(float(y.sum()) - 1.0) < 1e-5 and y[0] < y[1] < y[2] and (y > 0).all()
    x = np.random.default_rng(4).normal(0, 3, (6, 17)).astype(np.float32)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(oracle.softmax_f32(x), e / e.sum(axis=1, keepdims=True), rtol=1e-6, atol=0)


def test_gemm_tb_is_unfused_and_transposed():
    # B given as [n][k]; each step rounds the product before the add: after
    # -(1 + 2^-11), the product (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 rounds to
    # 1 + 2^-11 and the sum is 0; an fma keeps the 2^-24
    a = np.array([[-1.0, 1 + 2.0 ** -12]], np.float32)
    b = np.array([[1 + 2.0 ** -11, 1 + 2.0 ** -12]], np.float32)
    assert float(oracle.gemm_tb(a, b)[0, 0]) == 0.0
    assert float(oracle.gemm_f32(a, b.T.copy())[0, 0]) == 2.0 ** -24


def test_classifier_head_graph_matches_f64():
    # GlobalAveragePool -> Flatten -> Gemm(trans_b, bias) on the oracle's
    # CpuGraph against a float64 evaluation (catches a transposed weight)
    import __graft_entry__
    __graft_entry__.import_pkg()
    from dragonwing_edge_rs_amd.graph import Graph, GRAPH_F32
    from oracle.cpu_graph import CpuGraph
    r = np.random.default_rng(1)
    n, h, w, c, k = 3, 5, 5, 16, 12
    x = r.normal(0, 1, (n, h, w, c)).astype(np.float32)
    wt = r.normal(0, 0.1, (k, c)).astype(np.float32)
    b = r.normal(0, 0.1, (k,)).astype(np.float32)
    g = Graph(GRAPH_F32)
    g.add_tensor("x", x.shape, "f32")
    g.add_tensor("pool", (n, 1, 1, c), "f32")
    g.add_tensor("flat", (n, c), "f32")
    g.add_initializer("w", wt, "f32")
    g.add_initializer("b", b, "f32")
    g.add_tensor("y", (n, k), "f32")
    g.add_op("gap", "GlobalAveragePool", ["x"], ["pool"])
    g.add_op("flatten", "Flatten", ["pool"], ["flat"])
    g.add_op("fc", "Gemm", ["flat", "w", "b"], ["y"], trans_b=1)
    g.set_io(["x"], ["y"])
    cg = CpuGraph(g.to_dict(), g.initializer)
    cg.set_input("x", x)
    ref = x.astype(np.float64).mean(axis=(1, 2)) @ wt.T.astype(np.float64) + b
    np.testing.assert_allclose(cg.run()["y"], ref, rtol=0, atol=1e-5)
