"""YOLOv8n-shaped detection graph, built the way an ONNX export would arrive
at dragonwing-onnx: NCHW tensors, Conv (no bias) + BatchNormalization +
Sigmoid + Mul for every Conv module, C2f blocks (split / bottlenecks /
concat), SPPF (three cascaded 5x5 stride-1 max pools), a PAN neck with
nearest 2x upsampling, and a decoupled 3-scale detect head (box: 4*16 DFL
channels, cls: 80), whose last 1x1 convs carry a bias and no activation.

Topology: depth 0.33 / width 0.25 (the "n" scale): C2f at widths
32/64/128/256 with depths 1/2/2/1, 63 convolutions.  Weights are random
(no checkpoint): W ~ U[-sqrt(3/fan_in), +sqrt(3/fan_in)], BN gamma U[0.5,1.5],
beta and mean U[-0.1,0.1], var U[0.5,1.5], eps 1e-3, head biases
U[-0.1,0.1], all from the reference LCG.  The same structure is what
crates/dragonwing-test/src/yolo_e2e.rs:40-182 builds in miniature.
"""
from __future__ import annotations

import numpy as np

from . import synth
from .graph import GRAPH_F32, Graph

WIDTHS = (16, 32, 64, 128, 256)
NC, REG_MAX = 80, 16


class _Builder:
    def __init__(self, batch: int, size: int, seed: int):
        self.g = Graph(GRAPH_F32)
        self.r = synth.Rng(seed)
        self.batch = batch
        self.n_convs = 0
        self.n_params = 0
        self.shapes = {}
        self.f16_keep = []  # convs that stay fp16 in the int8 graph

    def tensor(self, name, c, h, w):
        self.g.add_tensor(name, (self.batch, c, h, w))
        self.shapes[name] = (c, h, w)
        return name

    def init(self, name, arr):
        self.g.add_initializer(name, arr.astype(np.float32))
        self.n_params += arr.size
        return name

    def conv_raw(self, name, x, c2, k, s, bias: bool):
        c1, h, w = self.shapes[x]
        p = k // 2
        ho, wo = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
        fan_in = c1 * k * k
        a = float(np.sqrt(3.0 / fan_in))
        wt = self.init(name + ".weight", self.r.uniform((c2, c1, k, k), -a, a))
        ins = [x, wt]
        if bias:
            ins.append(self.init(name + ".bias", self.r.uniform((c2,), -0.1, 0.1)))
        y = self.tensor(name + ".conv_out", c2, ho, wo)
        self.g.add_op(name, "Conv", ins, [y], kernel_shape=(k, k), strides=(s, s), pads=(p, p, p, p))
        self.n_convs += 1
        return y

    def conv(self, name, x, c2, k=1, s=1):
        """ultralytics Conv: Conv2d(bias=False) + BatchNorm2d + SiLU."""
        y = self.conv_raw(name, x, c2, k, s, bias=False)
        c, h, w = self.shapes[y]
        gam = self.init(name + ".bn.weight", self.r.uniform((c,), 0.5, 1.5))
        beta = self.init(name + ".bn.bias", self.r.uniform((c,), -0.1, 0.1))
        mean = self.init(name + ".bn.running_mean", self.r.uniform((c,), -0.1, 0.1))
        var = self.init(name + ".bn.running_var", self.r.uniform((c,), 0.5, 1.5))
        yb = self.tensor(name + ".bn_out", c, h, w)
        self.g.add_op(name + ".bn", "BatchNormalization", [y, gam, beta, mean, var], [yb], epsilon=1e-3)
        sg = self.tensor(name + ".sigmoid", c, h, w)
        self.g.add_op(name + ".act_sigmoid", "Sigmoid", [yb], [sg])
        out = self.tensor(name + ".out", c, h, w)
        self.g.add_op(name + ".act_mul", "Mul", [yb, sg], [out])
        return out

    def concat(self, name, xs):
        c = sum(self.shapes[x][0] for x in xs)
        _, h, w = self.shapes[xs[0]]
        y = self.tensor(name, c, h, w)
        self.g.add_op(name, "Concat", xs, [y], axis=1)
        return y

    def c2f(self, name, x, c2, n, shortcut):
        c = c2 // 2
        y = self.conv(name + ".cv1", x, 2 * c, 1, 1)
        _, h, w = self.shapes[y]
        a = self.tensor(name + ".split0", c, h, w)
        b = self.tensor(name + ".split1", c, h, w)
        self.g.add_op(name + ".split", "Split", [y], [a, b], axis=1, split_sizes=(c, c))
        ys = [a, b]
        for i in range(n):
            m = f"{name}.m{i}"
            t = self.conv(m + ".cv1", ys[-1], c, 3, 1)
            t = self.conv(m + ".cv2", t, c, 3, 1)
            if shortcut:
                s = self.tensor(m + ".add", c, h, w)
                self.g.add_op(m + ".add", "Add", [ys[-1], t], [s])
                t = s
            ys.append(t)
        cat = self.concat(name + ".cat", ys)
        return self.conv(name + ".cv2", cat, c2, 1, 1)

    def sppf(self, name, x, c2, k=5):
        c1, h, w = self.shapes[x]
        c_ = c1 // 2
        y = [self.conv(name + ".cv1", x, c_, 1, 1)]
        for i in range(3):
            t = self.tensor(f"{name}.pool{i}", c_, h, w)
            p = k // 2
            self.g.add_op(f"{name}.pool{i}", "MaxPool", [y[-1]], [t], kernel_shape=(k, k), strides=(1, 1),
                          pads=(p, p, p, p))
            y.append(t)
        return self.conv(name + ".cv2", self.concat(name + ".cat", y), c2, 1, 1)

    def upsample(self, name, x):
        c, h, w = self.shapes[x]
        y = self.tensor(name, c, 2 * h, 2 * w)
        self.g.add_op(name, "Resize", [x], [y], out_hw=(2 * h, 2 * w), mode="nearest")
        return y

    def detect(self, feats):
        c2 = max(16, self.shapes[feats[0]][0] // 4, 4 * REG_MAX)
        c3 = max(self.shapes[feats[0]][0], min(NC, 100))
        outs = []
        for i, f in enumerate(feats):
            bx = self.conv(f"det{i}.box0", f, c2, 3, 1)
            bx = self.conv(f"det{i}.box1", bx, c2, 3, 1)
            bx = self.conv_raw(f"det{i}.box2", bx, 4 * REG_MAX, 1, 1, bias=True)
            cl = self.conv(f"det{i}.cls0", f, c3, 3, 1)
            cl = self.conv(f"det{i}.cls1", cl, c3, 3, 1)
            cl = self.conv_raw(f"det{i}.cls2", cl, NC, 1, 1, bias=True)
            self.f16_keep += [f"det{i}.box2", f"det{i}.cls2"]
            outs.append(self.concat(f"out{i}", [bx, cl]))
        return outs


def build_yolov8n(batch: int = 32, size: int = 640, seed: int | None = None):
    """Returns (Graph, info): the NCHW float graph before any pass.

    info: input name, output names, conv count, parameter count, and the
    names of the convolutions that stay fp16 in the int8 graph (the stem and
    the head's last 1x1 convolutions)."""
    if size % 32:
        raise ValueError("input size must be a multiple of 32")
    b = _Builder(batch, size, synth.seed_for(3) if seed is None else seed)
    x = b.tensor("images", 3, size, size)
    w = WIDTHS
    t = b.conv("b0", x, w[0], 3, 2)
    b.f16_keep.append("b0")
    t = b.conv("b1", t, w[1], 3, 2)
    t = b.c2f("b2", t, w[1], 1, True)
    t = b.conv("b3", t, w[2], 3, 2)
    p3 = b.c2f("b4", t, w[2], 2, True)
    t = b.conv("b5", p3, w[3], 3, 2)
    p4 = b.c2f("b6", t, w[3], 2, True)
    t = b.conv("b7", p4, w[4], 3, 2)
    t = b.c2f("b8", t, w[4], 1, True)
    p5 = b.sppf("b9", t, w[4])
    t = b.upsample("n10", p5)
    t = b.concat("n11", [t, p4])
    n12 = b.c2f("n12", t, w[3], 1, False)
    t = b.upsample("n13", n12)
    t = b.concat("n14", [t, p3])
    o3 = b.c2f("n15", t, w[2], 1, False)
    t = b.conv("n16", o3, w[2], 3, 2)
    t = b.concat("n17", [t, n12])
    o4 = b.c2f("n18", t, w[3], 1, False)
    t = b.conv("n19", o4, w[3], 3, 2)
    t = b.concat("n20", [t, p5])
    o5 = b.c2f("n21", t, w[4], 1, False)
    outs = b.detect([o3, o4, o5])
    b.g.set_io([x], outs)
    info = {"input": x, "outputs": outs, "convs": b.n_convs, "params": b.n_params,
            "keep_f16": list(b.f16_keep), "batch": batch, "size": size,
            "out_shapes": [(batch,) + b.shapes[o][1:] + (b.shapes[o][0],) for o in outs]}
    return b.g, info


def conv_params(g_info_graph: Graph) -> int:
    """Number of weight + bias values after BN folding (for reporting)."""
    d = g_info_graph.to_dict()
    return sum(int(np.prod(t["dims"])) for n, t in d["tensors"].items()
               if t["init"] and (n.endswith(".weight") or n.endswith(".bias") or n.endswith("_bias_folded")))


def input_images(batch: int, size: int, index: int = 3) -> np.ndarray:
    """uniform[0,1] images, generated NCHW and returned NHWC f32."""
    r = synth.Rng(synth.seed_for(100 + index))
    x = r.uniform((batch, 3, size, size), 0.0, 1.0)
    return np.ascontiguousarray(x.transpose(0, 2, 3, 1))


def calibration_images(count: int = 16, size: int = 640, index: int = 4) -> np.ndarray:
    r = synth.Rng(synth.seed_for(200 + index))
    x = r.uniform((count, 3, size, size), 0.0, 1.0)
    return np.ascontiguousarray(x.transpose(0, 2, 3, 1))


def f16_graph(batch: int = 32, size: int = 640, seed: int | None = None):
    """The fp16 graph: fold_batchnorm -> NHWC -> f16 initializers."""
    g, info = build_yolov8n(batch, size, seed)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    g.convert_to_f16()
    return g, info


def int8_graph_from_ranges(ranges: dict, batch: int = 32, size: int = 640, seed: int | None = None):
    """The u8 QDQ graph at `batch` from previously calibrated ranges."""
    g, info = build_yolov8n(batch, size, seed)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    for n, (lo, hi) in ranges.items():
        g.set_activation_range(n, lo, hi)
    g.quantize_qdq(info["keep_f16"])
    info["ranges"] = ranges
    return g, info


def calibration_graph(batch: int, size: int = 640, seed: int | None = None):
    """The F32 NHWC graph calibration runs on: fold_batchnorm -> NHWC."""
    g, info = build_yolov8n(batch, size, seed)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    return g, info


def int8_graph(backend, batch: int = 32, size: int = 640, calib: np.ndarray | None = None,
               seed: int | None = None, calib_batch: int | None = None):
    """The u8 QDQ graph: calibrate the F32 graph on the GPU over `calib`
    (default: 16 uniform images), then quantize at `batch`.  The stem and
    the head's final 1x1 convs stay fp16."""
    from .graph import calibrate

    if calib is None:
        calib = calibration_images(16, size)
    cb = calib_batch or calib.shape[0]
    gc, info = build_yolov8n(cb, size, seed)
    gc.fold_batchnorm()
    gc.convert_nchw_to_nhwc()
    calibrate(backend, gc, info["input"], calib)
    ranges = {n: t["range"] for n, t in gc.to_dict()["tensors"].items() if "range" in t}
    g, info = build_yolov8n(batch, size, seed)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    for n, (lo, hi) in ranges.items():
        g.set_activation_range(n, lo, hi)
    g.quantize_qdq(info["keep_f16"])
    info["ranges"] = ranges
    return g, info


def add_detect_tail(g: Graph, info: dict, name: str = "output0", keep_heads: bool = False) -> str:
    """Appends the exported detect tail (DFL, dist2bbox, sigmoid, concat) to a
    finished f16 or u8 graph whose outputs are the three per-level head
    tensors: one YoloDetect op writing [batch, 4 + NC, A] f32, which becomes
    the graph's output (after the head tensors with keep_heads).  Strides
    8, 16, 32 (input size over level size)."""
    outs = info["outputs"]
    d = g.to_dict()["tensors"]
    size = info["size"]
    levels = [d[o]["dims"] for o in outs]  # NHWC after the passes
    A = sum(h * w for _, h, w, _ in levels)
    strides = [size // h for _, h, _, _ in levels]
    g.add_tensor(name, (info["batch"], 4 + NC, A), "f32")
    g.add_op("detect_tail", "YoloDetect", list(outs), [name], reg_max=REG_MAX, level_strides=strides)
    g.set_io([info["input"]], (list(outs) if keep_heads else []) + [name])
    return name
