"""The oracle's YOLOv8 detect tail and post-processing (oracle/dw_oracle.cpp
Part C) pinned on the CPU:

* iou, nms and postprocess_yolo against the reference's own tests
  (crates/dragonwing-onnx/src/postprocess.rs:310-407) and its end-to-end
  fixture (crates/dragonwing-test/src/yolo_e2e.rs:185-309), with the
  expected boxes worked out by hand;
* the order the reference returns (stable sort by confidence, then
  swap_remove of the suppressed entries from the back) on a hand-made case
  where that order is not the sorted one;
* greedy NMS by its defining invariants on random boxes: no two survivors of
  one class overlap above the threshold, and every suppressed box overlaps a
  higher-ranked survivor of its class above it;
* the detect tail by closed forms (uniform logits give the expectation 7.5
  exactly; a dominant bin gives its index; anchors at cell centres times the
  stride; sigmoid(0) = 1/2) and against an independent float64 evaluation of
  the ultralytics formulas.
"""
import numpy as np
import pytest

import oracle


def det(x1, y1, x2, y2, cls, conf):
    return (x1, y1, x2, y2, cls, conf)


def raw_from(dets, nc=80, A=8400):
    """[1, 4 + nc, A] raw output holding (cx, cy, w, h, cls, conf) at anchors."""
    raw = np.zeros((1, 4 + nc, A), np.float32)
    for a, (cx, cy, w, h, cls, conf) in dets.items():
        raw[0, 0:4, a] = (cx, cy, w, h)
        raw[0, 4 + cls, a] = conf
    return raw


def as_tuples(d):
    return [tuple(map(float, r["bbox"])) + (int(r["class_id"]), float(r["confidence"])) for r in d]


def test_iou_reference_cases():
    # test_iou_no_overlap / full_overlap / partial_overlap (postprocess.rs:310-330)
    assert oracle.iou([0, 0, 10, 10], [20, 20, 30, 30]) == 0.0
    assert abs(oracle.iou([0, 0, 10, 10], [0, 0, 10, 10]) - 1.0) < 1e-5
    assert abs(oracle.iou([0, 0, 10, 10], [5, 0, 15, 10]) - 50.0 / 150.0) < 1e-5
    # degenerate boxes: empty union gives 0
    assert oracle.iou([1, 1, 1, 1], [1, 1, 1, 1]) == 0.0


def test_e2e_fixture_postprocess():
    # create_synthetic_yolo_output + test_yolo_postprocess (yolo_e2e.rs:185-236):
    # 640x480 image, conf 0.25, IoU 0.45; person (0.9), car (0.85), and an
    # overlapping person (0.7) that NMS removes.
    raw = raw_from({0: (320, 240, 100, 200, 0, 0.9), 100: (500, 300, 150, 80, 2, 0.85),
                    1: (330, 245, 95, 195, 0, 0.7)})
    got = oracle.yolo_postprocess(raw, 640, 480, 0.25, 0.45)[0]
    # scale_x = 640/640, scale_y = 480/640 = 0.75 (postprocess.rs:97-100)
    assert as_tuples(got) == [
        (270.0, 105.0, 370.0, 255.0, 0, np.float32(0.9)),
        (425.0, 195.0, 575.0, 255.0, 2, np.float32(0.85)),
    ]


def test_nms_reference_cases():
    # test_nms_basic (postprocess.rs:333-347) and test_nms_different_classes
    # (:349-360), through the raw layout at 640x640 (scale 1)
    raw = raw_from({0: (5, 5, 10, 10, 0, 0.9), 1: (6, 6, 10, 10, 0, 0.8), 2: (25, 25, 10, 10, 0, 0.7)})
    got = oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.5)[0]
    assert len(got) == 2 and abs(float(got[0]["confidence"]) - 0.9) < 1e-5
    raw = raw_from({0: (5, 5, 10, 10, 0, 0.9), 1: (5, 5, 10, 10, 1, 0.8)})
    assert len(oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.5)[0]) == 2
    # agnostic: the same pair collapses to one
    assert len(oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.5, agnostic=True)[0]) == 1


def test_reference_output_order_after_swap_remove():
    # sorted: A(.9) B(.8, overlaps A) C(.7) D(.6); keep A, C, D.  Removing B by
    # swap_remove moves D into its slot: the reference returns A, D, C.
    raw = raw_from({10: (50, 50, 20, 20, 0, 0.9), 11: (51, 50, 20, 20, 0, 0.8),
                    12: (200, 200, 20, 20, 0, 0.7), 13: (400, 400, 20, 20, 0, 0.6)})
    got = as_tuples(oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.45)[0])
    assert [round(g[5], 6) for g in got] == [0.9, 0.6, 0.7]
    # ties keep anchor order (stable sort): two equal confidences, no overlap
    raw = raw_from({7: (300, 300, 10, 10, 3, 0.5), 3: (100, 100, 10, 10, 3, 0.5)})
    got = as_tuples(oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.45)[0])
    assert [g[0] for g in got] == [95.0, 295.0]


def test_threshold_and_class_choice():
    # best class by strict '>', from (0, 0.0): an equal later score does not win;
    # conf exactly at the threshold is kept (skip only when below)
    raw = raw_from({0: (50, 50, 10, 10, 3, 0.25)})
    raw[0, 4 + 7, 0] = 0.25
    got = as_tuples(oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.45)[0])
    assert len(got) == 1 and got[0][4] == 3
    assert oracle.yolo_postprocess(raw, 640, 640, 0.2500001, 0.45)[0].size == 0
    # clamped corners
    raw = raw_from({0: (5, 630, 40, 40, 1, 0.9)})
    got = as_tuples(oracle.yolo_postprocess(raw, 640, 640, 0.25, 0.45)[0])
    assert got[0][:4] == (0.0, 610.0, 25.0, 640.0)


@pytest.mark.parametrize("agnostic", [False, True])
def test_nms_invariants_random(agnostic):
    rng = np.random.default_rng(11)
    nc, A = 5, 600
    raw = np.zeros((1, 4 + nc, A), np.float32)
    raw[0, 0] = rng.uniform(0, 640, A)
    raw[0, 1] = rng.uniform(0, 640, A)
    raw[0, 2] = rng.uniform(5, 120, A)
    raw[0, 3] = rng.uniform(5, 120, A)
    raw[0, 4:] = rng.uniform(0, 1, (nc, A))
    got = oracle.yolo_postprocess(raw, 640, 640, 0.3, 0.45, agnostic)[0]
    # every candidate above the threshold, from the raw data directly
    best = raw[0, 4:].argmax(0)
    conf = raw[0, 4:].max(0)
    cand = [(a, int(best[a]), float(conf[a])) for a in range(A) if conf[a] >= np.float32(0.3)]
    assert 0 < len(got) < len(cand)
    kept = as_tuples(got)
    same = (lambda c1, c2: True) if agnostic else (lambda c1, c2: c1 == c2)
    for i in range(len(kept)):
        for j in range(i + 1, len(kept)):
            if same(kept[i][4], kept[j][4]):
                assert oracle.iou(kept[i][:4], kept[j][:4]) <= np.float32(0.45)
    kept_set = {(k[4], k[5], k[:4]) for k in kept}
    for a, c, cf in cand:
        cx, cy, w, h = raw[0, 0:4, a]
        hw, hh = np.float32(w) / np.float32(2), np.float32(h) / np.float32(2)
        box = tuple(float(min(max(np.float32(v), np.float32(0)), np.float32(640)))
                    for v in (cx - hw, cy - hh, cx + hw, cy + hh))
        if (c, cf, box) in kept_set:
            continue
        # suppressed: some survivor ranked above it (higher confidence) overlaps it
        assert any(same(k[4], c) and k[5] >= cf and oracle.iou(k[:4], box) > np.float32(0.45) for k in kept)


def tail_levels(rng, n, sizes, nc=80, reg=16, scale=2.0):
    return [oracle.f16_from_f32(rng.normal(0, scale, (n, h, w, 4 * reg + nc)).astype(np.float32))
            for h, w in sizes]


def test_detect_tail_closed_forms():
    sizes = [(4, 6), (2, 3)]
    strides = [8.0, 16.0]
    lv = [np.zeros((1, h, w, 64 + 80), np.uint16) for h, w in sizes]  # all logits +0
    y = oracle.yolo_detect_tail_f16(lv, strides)
    A = 4 * 6 + 2 * 3
    assert y.shape == (1, 84, A)
    a = 0
    for (h, w), st in zip(sizes, strides):
        for gy in range(h):
            for gx in range(w):
                # uniform softmax: every distance is sum(k)/16 = 7.5 exactly
                assert y[0, 0, a] == (gx + 0.5) * st and y[0, 1, a] == (gy + 0.5) * st
                assert y[0, 2, a] == 15.0 * st and y[0, 3, a] == 15.0 * st
                a += 1
    assert np.all(y[0, 4:] == 0.5)
    # a dominant bin k0 per side: distance k0 (other bins weigh e^-40)
    lv = [np.zeros((1, 2, 2, 144), np.float32)]
    for j, k0 in enumerate((3, 0, 15, 9)):
        lv[0][..., j * 16 + k0] = 40.0
    y = oracle.yolo_detect_tail_f16([oracle.f16_from_f32(lv[0])], [32.0])
    d = np.array([3, 0, 15, 9], np.float64)
    for a, (gy, gx) in enumerate([(0, 0), (0, 1), (1, 0), (1, 1)]):
        x1, y1 = gx + 0.5 - d[0], gy + 0.5 - d[1]
        x2, y2 = gx + 0.5 + d[2], gy + 0.5 + d[3]
        want = np.array([(x1 + x2) / 2, (y1 + y2) / 2, x2 - x1, y2 - y1]) * 32
        np.testing.assert_allclose(y[0, :4, a], want, rtol=0, atol=1e-3)


def test_detect_tail_vs_float64():
    rng = np.random.default_rng(3)
    sizes, strides = [(8, 8), (4, 4), (2, 2)], [8.0, 16.0, 32.0]
    lv = tail_levels(rng, 2, sizes)
    y = oracle.yolo_detect_tail_f16(lv, strides)
    # independent float64 evaluation of DFL / dist2bbox / sigmoid
    cols = []
    for x, (h, w), st in zip(lv, sizes, strides):
        v = oracle.f16_to_f32(x).astype(np.float64).reshape(2, h * w, 144)
        box = v[..., :64].reshape(2, h * w, 4, 16)
        p = np.exp(box - box.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        dist = (p * np.arange(16)).sum(-1)
        gy, gx = np.divmod(np.arange(h * w), w)
        ax, ay = gx + 0.5, gy + 0.5
        x1, y1 = ax - dist[..., 0], ay - dist[..., 1]
        x2, y2 = ax + dist[..., 2], ay + dist[..., 3]
        b = np.stack([(x1 + x2) / 2, (y1 + y2) / 2, x2 - x1, y2 - y1], 1) * st
        c = 1 / (1 + np.exp(-v[..., 64:].transpose(0, 2, 1)))
        cols.append(np.concatenate([b, c], 1))
    ref = np.concatenate(cols, 2)
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=2e-5)
