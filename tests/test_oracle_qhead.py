"""The quantized classifier head in the oracle (QGemm u8 x s8 -> u8,
QLinearGlobalAveragePool) and in the QDQ quantizer, on the CPU.

QGemm is the oracle's QLinearConv on a 1x1 kernel over the rows of A; it is
checked against an independent numpy evaluation of the definition (int64
sums, f32 multiply by M[j] = a_s * b_s[j] / y_s, round half to even,
saturation), with exact .5 ties and both orientations of B.
QLinearGlobalAveragePool against the same kind of evaluation and closed
forms: a constant image averages to its value; ties at x.5 round to even."""
import numpy as np
import pytest

import oracle


def qgemm_numpy(a, b, bias, a_s, a_zp, b_s, y_s, y_zp):
    acc = (a.astype(np.int64) - a_zp) @ b.astype(np.int64)
    if bias is not None:
        acc = acc + bias.astype(np.int64)
    m = (np.float32(a_s) * b_s.astype(np.float32)) / np.float32(y_s)
    q = np.rint(acc.astype(np.int32).astype(np.float32) * m) + np.float32(y_zp)
    return np.clip(q, 0, 255).astype(np.uint8)


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("m,n,k,a_zp", [(4, 8, 16, 128), (3, 12, 32, 0), (5, 4, 48, 255)])
def test_qgemm_matches_definition(m, n, k, a_zp, trans_b):
    r = np.random.default_rng(m * n + k + a_zp)
    a = r.integers(0, 256, (m, k)).astype(np.uint8)
    b = r.integers(-127, 128, (k, n)).astype(np.int8)
    bias = r.integers(-4096, 4097, n).astype(np.int32)
    b_s = np.exp(r.uniform(np.log(1e-3), np.log(1e-2), n)).astype(np.float32)
    want = qgemm_numpy(a, b, bias, 0.02, a_zp, b_s, 0.05, 128)
    bb = np.ascontiguousarray(b.T) if trans_b else b
    got = oracle.qgemm_u8s8(a, bb, bias, 0.02, a_zp, b_s, 0.05, 128, trans_b=trans_b)
    np.testing.assert_array_equal(got, want)


def test_qgemm_ties_and_saturation():
    # M = 0.5 exactly (a_s 1, b_s 0.5, y_s 1): acc 5 -> 2.5 -> 2, acc 7 -> 3.5 -> 4,
    # acc -3 -> -1.5 -> -2; large sums saturate at 0 and 255
    a = np.array([[133, 128], [135, 128], [125, 128], [255, 255], [0, 0]], np.uint8)
    b = np.array([[1, 1, 1, 1], [0, 0, 0, 0]], np.int8)
    bs = np.full(4, 0.5, np.float32)
    y = oracle.qgemm_u8s8(a, b, None, 1.0, 128, bs, 1.0, 100)
    assert list(y[:, 0]) == [102, 104, 98, 164, 36]
    b2 = np.array([[127] * 4, [127] * 4], np.int8)
    y2 = oracle.qgemm_u8s8(a, b2, None, 1.0, 128, np.full(4, 1.0, np.float32), 1.0, 128)
    assert y2[3, 0] == 255 and y2[4, 0] == 0


def test_qlinear_gap_definition_and_closed_forms():
    r = np.random.default_rng(2)
    x = r.integers(0, 256, (3, 7, 7, 40)).astype(np.uint8)
    got = oracle.qlinear_gap_u8(x, 0.03, 120, 0.02, 131)
    acc = (x.astype(np.int64) - 120).sum(axis=(1, 2))
    mul = (np.float32(0.03) / np.float32(0.02)) / np.float32(49)
    want = np.clip(np.rint(acc.astype(np.float32) * mul) + 131, 0, 255).astype(np.uint8)
    np.testing.assert_array_equal(got, want)
    # a constant image averages to itself (same scale and zero point)
    c = np.full((1, 7, 7, 3), 200, np.uint8)
    assert list(oracle.qlinear_gap_u8(c, 0.1, 128, 0.1, 128)[0]) == [200] * 3
    # 2 x 2 image, sums 2 and 6 over 4 pixels: 0.5 -> 0, 1.5 -> 2 (half to even)
    t = np.array([[[[129], [129]], [[128], [128]]], [[[129], [130]], [[131], [130]]]], np.uint8)
    assert list(oracle.qlinear_gap_u8(t, 1.0, 128, 1.0, 0)[:, 0]) == [0, 2]


def test_quantizer_turns_the_head_into_qgemm():
    import __graft_entry__
    __graft_entry__.import_pkg()
    from dragonwing_edge_rs_amd.graph import Graph, GRAPH_F32
    r = np.random.default_rng(0)
    g = Graph(GRAPH_F32)
    g.add_tensor("x", (2, 4, 4, 32))
    g.add_tensor("pool", (2, 1, 1, 32))
    g.add_tensor("flat", (2, 32))
    g.add_initializer("w", r.normal(0, 0.1, (12, 32)).astype(np.float32))
    g.add_initializer("b", r.normal(0, 0.1, 12).astype(np.float32))
    g.add_tensor("y", (2, 12))
    g.add_op("gap", "GlobalAveragePool", ["x"], ["pool"])
    g.add_op("flatten", "Flatten", ["pool"], ["flat"])
    g.add_op("fc", "Gemm", ["flat", "w", "b"], ["y"], trans_b=1)
    g.set_io(["x"], ["y"])
    for name, rng in (("x", (-2.0, 3.0)), ("pool", (-0.5, 0.7)), ("flat", (-0.5, 0.7)), ("y", (-1.0, 1.5))):
        g.set_activation_range(name, *rng)
    wt = g.initializer("w", np.float32, (12, 32)).copy()
    g.quantize_qdq()
    d = g.to_dict()
    types = [op["type"] for op in d["ops"]]
    assert types == ["QuantizeLinear", "QLinearGlobalAveragePool", "Flatten", "QGemm"], types
    t = d["tensors"]
    assert t["w"]["dims"] == [1, 1, 32, 12] and t["b"]["dtype"] == 4
    assert t["pool"]["scale"] == t["flat"]["scale"]  # Flatten moves bytes only
    # weights per output column: |w| max / 127, and transposed into [k][n]
    ws = np.array(t["w"]["ch_scales"], np.float32)
    np.testing.assert_array_equal(ws, np.abs(wt).max(axis=1) / np.float32(127))
    wq = g.initializer("w", np.int8, (32, 12))
    np.testing.assert_array_equal(wq, np.clip(np.round(wt.T * (np.float32(1) / ws)), -128, 127).astype(np.int8))
