"""Pins the oracle's Part D (layout ops, broadcasting, average pool):

* the reference's known answers: transpose_f32 NCHW -> NHWC (ops.rs:1032-1046),
  sub_f32 / div_f32 on the reference's own vectors (ops.rs:1049-1100),
  avgpool2d of ones (ops.rs:741-762);
* transpose and slice against explicit index loops on small tensors, and
  the f16 round trip through f32 that the reference's dispatch applies
  (subnormals halved, dtype.rs:236-248); a pure layout transpose keeps the
  bits;
* broadcasting against the reference's modular rule b[i % len(b)]
  (runtime.rs:1045-1860) computed with explicit loops, f16 operands
  decoded with the reference decode and every result a single rounding
  of the exact f64 operation (one IEEE f32 operation, then f16 RNE);
* average pool against f64 window means, with the f32 summation order
  (ph then pw) shown to matter on an adversarial window.
"""
import itertools

import numpy as np

import oracle


def test_transpose_reference_known_answer():  # ops.rs:1032-1046
    x = np.arange(24, dtype=np.float32).reshape(1, 2, 3, 4)
    y = oracle.transpose(x, (0, 2, 3, 1))
    assert y.shape == (1, 3, 4, 2) and y.ravel()[0] == 0.0 and y.ravel()[1] == 12.0


def test_transpose_matches_index_loops():
    r = np.random.default_rng(5)
    x = r.normal(size=(2, 3, 4, 5)).astype(np.float32)
    for perm in itertools.permutations(range(4)):
        y = oracle.transpose(x, perm)
        for idx in [(0, 0, 0, 0), (1, 2, 3, 4), (1, 0, 2, 3), (0, 1, 1, 2)]:
            src = [0] * 4
            out_idx = tuple(idx[k] % y.shape[k] for k in range(4))
            for k in range(4):
                src[perm[k]] = out_idx[k]
            assert y[out_idx] == x[tuple(src)]
    # rank 3 (the DFL layout): perm over three axes
    z = r.normal(size=(2, 6, 7)).astype(np.float32)
    np.testing.assert_array_equal(oracle.transpose(z, (0, 2, 1))[1, 3, 4], z[1, 4, 3])


def test_transpose_f16_round_trip():
    h = np.array([[0x0002, 0x3C00], [0x8004, 0x03FF]], np.uint16)
    # the reference's f16 Transpose: subnormals come back halved
    np.testing.assert_array_equal(oracle.transpose(h, (1, 0)), [[0x0001, 0x8002], [0x3C00, 0x0200]])
    # a layout transpose moves the bits unchanged
    np.testing.assert_array_equal(oracle.transpose(h, (1, 0), f16_round_trip=False), h.T)


def test_slice_matches_index_loops():
    x = np.arange(2 * 7 * 5 * 3, dtype=np.float32).reshape(2, 7, 5, 3)
    y = oracle.slice_axes(x, [(1, 2, 7, 2), (3, 1, 3, 1)])
    assert y.shape == (2, 3, 5, 2)
    for n, i, j, c in itertools.product(range(2), range(3), range(5), range(2)):
        assert y[n, i, j, c] == x[n, 2 + 2 * i, j, 1 + c]
    h = np.array([0x0002, 0x3C00, 0x0006], np.uint16)
    np.testing.assert_array_equal(oracle.slice_axes(h, [(0, 0, 3, 2)]), [0x0001, 0x0003])


def test_sub_div_reference_known_answers():  # ops.rs:1049-1100
    a = np.arange(100, dtype=np.float32) * 2
    b = np.arange(100, dtype=np.float32) * 0.5
    np.testing.assert_array_equal(oracle.binary("Sub", a, b), a - b)
    a = np.arange(1, 101, dtype=np.float32) * 2
    b = np.arange(1, 101, dtype=np.float32) * 0.5
    np.testing.assert_array_equal(oracle.binary("Div", a, b), np.full(100, 4.0, np.float32))


def modular(op, a, b):
    """The reference's broadcast loop: out[i] = a[i] op b[i % len(b)]."""
    af, bf = a.ravel().astype(np.float64), b.ravel().astype(np.float64)
    out = np.empty(af.size)
    for i in range(af.size):
        x, y = af[i], bf[i % bf.size]
        out[i] = {"Add": x + y, "Sub": x - y, "Mul": x * y, "Div": x / y}[op]
    return out.reshape(a.shape)


def test_broadcast_matches_modular_rule_and_single_rounding():
    r = np.random.default_rng(9)
    a = r.normal(size=(2, 4, 30)).astype(np.float32)
    for b in (r.normal(size=(30,)).astype(np.float32), r.normal(size=(4, 30)).astype(np.float32) + 2,
              np.array([3.0], np.float32)):
        for op in ("Add", "Sub", "Mul", "Div"):
            got = oracle.binary(op, a, b.reshape((1,) * (3 - b.ndim) + b.shape))
            # one f32 rounding of the exact operation (f64 holds the exact
            # result of +, -, * of two f32; the quotient rounds once more,
            # which cannot move a result off its f32 rounding)
            np.testing.assert_array_equal(got, modular(op, a, b).astype(np.float32), err_msg=op)
    # a smaller first operand (anchor points - distances)
    anchors = r.uniform(0, 80, size=(1, 2, 30)).astype(np.float32)
    lt = r.uniform(0, 5, size=(3, 2, 30)).astype(np.float32)
    got = oracle.binary("Sub", anchors, lt)
    assert got.shape == (3, 2, 30)
    np.testing.assert_array_equal(got[2], (anchors[0].astype(np.float64) - lt[2]).astype(np.float32))


def test_binary_f16_rounding_points():
    r = np.random.default_rng(10)
    a = oracle.f16_from_f32(r.normal(size=4000).astype(np.float32))
    b = oracle.f16_from_f32(r.normal(size=4000).astype(np.float32) + 3)
    a[:4] = [0x0003, 0x8001, 0x03FF, 0x0200]  # subnormals: decoded at half value
    dec = lambda h: np.where(((h & 0x7C00) == 0) & ((h & 0x3FF) != 0),
                             h.view(np.float16).astype(np.float64) * 0.5, h.view(np.float16).astype(np.float64))
    for op in ("Add", "Sub", "Mul", "Div"):
        exact = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide}[op](dec(a), dec(b))
        want = exact.astype(np.float32).astype(np.float16).view(np.uint16)  # f32 once, then f16 RNE
        np.testing.assert_array_equal(oracle.binary(op, a, b), want, err_msg=op)


def test_avgpool_reference_known_answer_and_means():  # ops.rs:741-762
    np.testing.assert_array_equal(oracle.avgpool2d_nhwc(np.ones((1, 4, 4, 1), np.float32), (2, 2), (2, 2)), 1.0)
    r = np.random.default_rng(11)
    x = r.normal(size=(2, 9, 7, 3)).astype(np.float32)
    y = oracle.avgpool2d_nhwc(x, (3, 2), (2, 1))
    assert y.shape == (2, 4, 6, 3)
    ref = np.array([[[[x[n, 2 * i:2 * i + 3, j:j + 2, c].astype(np.float64).mean() for c in range(3)]
                      for j in range(6)] for i in range(4)] for n in range(2)])
    assert np.max(np.abs(y - ref)) < 1e-6
    # the f32 sum runs in order (ph, pw): an order-sensitive window
    w = np.array([1e8, 1.0, -1e8, 1.0], np.float32).reshape(1, 2, 2, 1)
    assert oracle.avgpool2d_nhwc(w, (2, 2), (1, 1))[0, 0, 0, 0] == np.float32(0.25)  # ((1e8+1)-1e8+1)/4
