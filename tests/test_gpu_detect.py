"""GPU parity of the YOLOv8 detect tail and post-processing against the
oracle (oracle/dw_oracle.cpp Part C):

* the tail (DFL softmax + expectation, dist2bbox, sigmoid, concat) at the
  headline shape, batch 32 at 640x640 (levels 80x80, 40x40, 20x20 of 144
  channels): within 1e-5 of each output's scale (the fp32 bar is 1e-3; only
  expf differs between the device and the host libm), most values bit-equal;
* the tail as a graph op after the INT8 YOLOv8n graph at batch 32, 640x640,
  checked against the oracle on the graph's own head outputs;
* postprocess_yolo (decode + NMS) on the device: the detections of every
  image identical, bit for bit and in the reference's order, to the
  oracle's on the same raw output; the reference's end-to-end fixture; the
  class-agnostic variant; the capacity errors.
"""
import numpy as np
import pytest

import oracle
from dragonwing_edge_rs_amd import HipError, ops, yolo
from dragonwing_edge_rs_amd.graph import HipGraphRuntime

pytestmark = pytest.mark.gpu

SIZES = [(80, 80), (40, 40), (20, 20)]
STRIDES = [8.0, 16.0, 32.0]


def tail_err(got, ref):
    """max |got - ref| over each row's scale (per output channel), and the
    fraction of bit-equal values."""
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    scale = np.maximum(np.abs(r).max(axis=(0, 2), keepdims=True), 1e-30)
    return float((np.abs(g - r) / scale).max()), float(np.mean(got.view(np.uint32) == ref.view(np.uint32)))


def random_levels(rng, n):
    return [oracle.f16_from_f32(rng.normal(0, 3, (n, h, w, 144)).astype(np.float32)) for h, w in SIZES]


def run_tail(backend, levels, n):
    bufs = [backend.from_numpy(x) for x in levels]
    A = sum(h * w for h, w in SIZES)
    out = backend.alloc(n * 84 * A * 4)
    ops.yolo_detect_tail(backend, bufs, SIZES, STRIDES, n, out)
    return backend.to_numpy(out, np.float32, (n, 84, A))


def test_detect_tail_full_shape(backend):
    rng = np.random.default_rng(21)
    lv = random_levels(rng, 32)
    got = run_tail(backend, lv, 32)
    ref = oracle.yolo_detect_tail_f16(lv, STRIDES)
    err, same = tail_err(got, ref)
    print(f"detect tail b32 640: max scaled error {err:.2e}, bit-equal {same:.4f}")
    assert err <= 1e-5 and same > 0.5


def test_detect_tail_subnormal_and_extreme_inputs(backend):
    # f16 subnormals (decoded at half value by the reference), zeros, +-inf
    # logits, large magnitudes
    rng = np.random.default_rng(5)
    lv = random_levels(rng, 1)
    flat = lv[0].reshape(-1)
    flat[:200] = rng.integers(1, 0x400, 200).astype(np.uint16)  # positive subnormals
    flat[200:260] = 0x8000
    flat[300] = 0x7C00  # +inf class or box logit
    flat[301] = 0xFC00
    flat[400:500] = oracle.f16_from_f32(np.full(100, 60000.0, np.float32))
    got = run_tail(backend, lv, 1)
    ref = oracle.yolo_detect_tail_f16(lv, STRIDES)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    err, _ = tail_err(np.where(fin, got, 0), np.where(fin, ref, 0))
    assert err <= 1e-5


@pytest.fixture(scope="module")
def int8_tail_run(backend):
    g, info = yolo.int8_graph(backend, batch=32, size=640)
    name = yolo.add_detect_tail(g, info, keep_heads=True)
    x = yolo.input_images(32, 640)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    heads = [rt.get_output_bytes(o).view(np.uint16).reshape(s) for o, s in zip(info["outputs"], info["out_shapes"])]
    raw = rt.get_output_bytes(name).view(np.float32).reshape(32, 84, 8400)
    return heads, raw


def test_detect_tail_graph_op_int8_b32(int8_tail_run):
    heads, raw = int8_tail_run
    ref = oracle.yolo_detect_tail_f16(heads, STRIDES)
    err, same = tail_err(raw, ref)
    print(f"graph detect tail: max scaled error {err:.2e}, bit-equal {same:.4f}")
    assert err <= 1e-5


def compare_dets(got, ref):
    assert len(got) == len(ref)
    for b, (g, r) in enumerate(zip(got, ref)):
        assert g.shape == r.shape, f"image {b}: {g.shape[0]} vs {r.shape[0]} detections"
        assert g.tobytes() == r.tobytes(), f"image {b}: detections differ"


@pytest.mark.parametrize("conf,iou", [(0.25, 0.45), (0.4, 0.3)])
def test_postprocess_full_batch_bit_exact(backend, int8_tail_run, conf, iou):
    _, raw = int8_tail_run
    buf = backend.from_numpy(raw)
    got = ops.yolo_postprocess(backend, buf, 32, 80, 8400, 640, 640, conf, iou)
    ref = oracle.yolo_postprocess(raw, 640, 640, conf, iou)
    print(f"conf {conf} iou {iou}: detections per image {[len(r) for r in ref[:4]]} ...")
    assert all(len(r) > 0 for r in ref)
    compare_dets(got, ref)


def test_postprocess_agnostic_bit_exact(backend, int8_tail_run):
    _, raw = int8_tail_run
    sub = np.ascontiguousarray(raw[:3])
    buf = backend.from_numpy(sub)
    got = ops.yolo_postprocess(backend, buf, 3, 80, 8400, 640, 480, 0.3, 0.45, agnostic=True)
    ref = oracle.yolo_postprocess(sub, 640, 480, 0.3, 0.45, agnostic=True)
    print(f"agnostic: detections per image {[len(r) for r in ref]}")
    assert all(len(r) > 0 for r in ref)
    compare_dets(got, ref)


def test_postprocess_reference_fixture(backend):
    # create_synthetic_yolo_output (yolo_e2e.rs:185-221) on a 640x480 image
    raw = np.zeros((1, 84, 8400), np.float32)
    for a, (cx, cy, w, h, cls, cf) in {0: (320, 240, 100, 200, 0, 0.9), 100: (500, 300, 150, 80, 2, 0.85),
                                       1: (330, 245, 95, 195, 0, 0.7)}.items():
        raw[0, 0:4, a] = (cx, cy, w, h)
        raw[0, 4 + cls, a] = cf
    got = ops.yolo_postprocess(backend, backend.from_numpy(raw), 1, 80, 8400, 640, 480, 0.25, 0.45)
    ref = oracle.yolo_postprocess(raw, 640, 480, 0.25, 0.45)
    compare_dets(got, ref)
    assert [int(d["class_id"]) for d in got[0]] == [0, 2]


def test_postprocess_errors(backend):
    # more candidates over the threshold than one image's workgroup holds
    A = 9000
    raw = np.zeros((1, 84, A), np.float32)
    raw[0, 4] = 0.9
    raw[0, 2:4] = 4.0
    buf = backend.from_numpy(raw)
    with pytest.raises(HipError):
        ops.yolo_postprocess(backend, buf, 1, 80, A)
    # a capacity below the number of detections
    raw = np.zeros((1, 84, 64), np.float32)
    raw[0, 0] = np.arange(64) * 10.0
    raw[0, 2:4] = 2.0
    raw[0, 4] = 0.9
    buf = backend.from_numpy(raw)
    with pytest.raises(HipError):
        ops.yolo_postprocess(backend, buf, 1, 80, 64, cap=8)
    got = ops.yolo_postprocess(backend, buf, 1, 80, 64)
    compare_dets(got, oracle.yolo_postprocess(raw))
