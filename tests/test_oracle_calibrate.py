"""The oracle Calibrator (oracle/cpu_graph.py ``calibrate``; the reference's
Calibrator::feed / compute_params, crates/dragonwing-onnx/src/calibration.rs
:56-69, :170-260) pinned on the CPU against definitions that do not go
through it:

* ranges equal numpy min/max over each tensor of the graph run on the whole
  image set, computed here by independent means (a 1x1 identity conv whose
  output is its input, a ReLU, a closed-form bias);
* batches merge: calibrating 4 images two at a time equals one pass of 4;
* non-finite values are skipped (TensorStats::update, :56-63) and the graph
  input is not recorded (feed records op outputs only, :170-205);
* absmax/127 of the result is QuantScale::from_range (its KATs are in
  test_oracle_int8.py).

A calibrator that recorded the last batch only, kept NaN/inf, recorded the
graph input or mixed up min and max fails one of these."""
import numpy as np
import pytest

import oracle
from oracle.cpu_graph import calibrate

from dragonwing_edge_rs_amd.graph import GRAPH_F32, Graph


def identity_relu_graph(n, h, w, c, bias):
    """x -> Conv 1x1 (identity weights, bias) -> Relu, NHWC f32."""
    g = Graph(GRAPH_F32)
    g.add_tensor("x", (n, h, w, c))
    g.add_initializer("w", np.eye(c, dtype=np.float32).reshape(1, 1, c, c))
    g.add_initializer("b", np.asarray(bias, np.float32))
    g.add_tensor("y", (n, h, w, c))
    g.add_op("conv", "Conv", ["x", "w", "b"], ["y"], kernel_shape=(1, 1))
    g.add_tensor("r", (n, h, w, c))
    g.add_op("relu", "Relu", ["y"], ["r"])
    g.set_io(["x"], ["r"])
    return g


def run_calibrate(g, images):
    return calibrate(g.to_dict(), g.initializer, "x", images)


def test_ranges_are_min_max_over_all_images():
    rng = np.random.default_rng(5)
    c = 4
    bias = np.array([0.5, -0.25, 0.0, 2.0], np.float32)
    imgs = rng.uniform(-3, 3, (4, 3, 5, c)).astype(np.float32)
    # one image holds the extremes of the whole set
    imgs[2, 1, 1, 0] = -7.5
    imgs[3, 0, 4, 3] = 9.25
    g = identity_relu_graph(2, 3, 5, c, bias)
    st = run_calibrate(g, imgs)
    assert set(st) == {"y", "r"}  # op outputs only: the graph input is not recorded
    # identity 1x1 conv: y = fma(x, 1, 0) + bias, exact in f32 for these values
    y = (imgs + bias).astype(np.float32)
    assert st["y"] == (float(y.min()), float(y.max()))
    r = np.maximum(y, 0)
    assert st["r"] == (float(r.min()), float(r.max()))
    # batches merge: the same images at batch 4 in one pass
    g4 = identity_relu_graph(4, 3, 5, c, bias)
    assert run_calibrate(g4, imgs) == st
    # the extremes sit in different batches: keeping either batch alone fails
    first, last = y[:2], y[2:]
    assert float(first.max()) < st["y"][1] and float(last.max()) == st["y"][1]
    assert float(first.min()) > st["y"][0] and float(last.min()) == st["y"][0]
    imgs_swapped = np.concatenate([imgs[2:], imgs[:2]])
    imgs_swapped[0, 1, 1, 0] = 0.0  # move the minimum into the first batch only
    imgs_swapped[2, 1, 1, 0] = -7.5
    assert run_calibrate(g, imgs_swapped)["y"][0] == st["y"][0]


def test_non_finite_values_are_skipped():
    c = 2
    imgs = np.zeros((2, 2, 2, c), np.float32)
    imgs[0, 0, 0, 0] = np.inf
    imgs[0, 0, 1, 0] = -np.inf
    imgs[1, 1, 1, 1] = np.nan
    imgs[1, 0, 0, 1] = 3.0
    imgs[0, 1, 1, 1] = -2.0
    g = identity_relu_graph(1, 2, 2, c, [0.0, 0.0])
    st = run_calibrate(g, imgs)
    assert st["y"] == (-2.0, 3.0)
    assert st["r"] == (0.0, 3.0)
    # the scale the quantizer takes from it: absmax / 127 (QuantScale::from_range)
    assert oracle.scale_from_range(*st["y"]) == np.float32(3.0) / np.float32(127.0)


def test_image_count_must_fill_batches():
    g = identity_relu_graph(2, 2, 2, 2, [0.0, 0.0])
    with pytest.raises(ValueError):
        run_calibrate(g, np.zeros((3, 2, 2, 2), np.float32))
