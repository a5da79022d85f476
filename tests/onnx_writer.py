"""A small ONNX writer for the tests: protobuf wire encoding of ModelProto,
GraphProto, NodeProto, TensorProto, ValueInfoProto and AttributeProto
(onnx.proto field numbers), with switches for the encodings a reader must
accept (raw_data or typed fields, packed or unpacked repeated ints,
symbolic dimensions).  Test infrastructure: no onnx package is installed.

Also: exporters from this repository's graph IR to ONNX, the float NCHW
graph as an exporter would write it, and a u8 graph in QDQ form."""
from __future__ import annotations

import struct

import numpy as np

# TensorProto.DataType
FLOAT, UINT8, INT8, INT32, INT64, FLOAT16 = 1, 2, 3, 6, 7, 10
NP_TYPE = {np.dtype(np.float32): FLOAT, np.dtype(np.uint8): UINT8, np.dtype(np.int8): INT8,
           np.dtype(np.int32): INT32, np.dtype(np.int64): INT64, np.dtype(np.float16): FLOAT16}


def varint(v: int) -> bytes:
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(num: int, wt: int) -> bytes:
    return varint((num << 3) | wt)


def f_varint(num: int, v: int) -> bytes:
    return key(num, 0) + varint(v)


def f_bytes(num: int, b: bytes) -> bytes:
    return key(num, 2) + varint(len(b)) + b


def f_str(num: int, s: str) -> bytes:
    return f_bytes(num, s.encode())


def f_float(num: int, x: float) -> bytes:
    return key(num, 5) + struct.pack("<f", x)


def f_ints(num: int, vals, packed=True) -> bytes:
    if packed:
        return f_bytes(num, b"".join(varint(int(v)) for v in vals))
    return b"".join(f_varint(num, int(v)) for v in vals)


def tensor(name: str, arr, raw=True, packed_dims=True) -> bytes:
    a = np.asarray(arr)
    a = np.ascontiguousarray(a) if a.ndim else a  # keep 0-d scalars 0-d
    out = f_ints(1, a.shape, packed_dims) if a.shape else b""
    out += f_varint(2, NP_TYPE[a.dtype])
    if raw:
        out += f_bytes(9, a.tobytes())
    elif a.dtype == np.float32:
        out += f_bytes(4, a.tobytes())  # float_data, packed fixed32
    elif a.dtype == np.int64:
        out += f_ints(7, a.ravel())
    else:  # int32_data: varints of the values (u8 / i8 / i32) or f16 bits
        vals = a.view(np.uint16) if a.dtype == np.float16 else a
        out += f_ints(5, vals.ravel().astype(np.int64))
    return out + f_str(8, name)


def attr(name: str, v) -> bytes:
    out = f_str(1, name)
    if isinstance(v, bool) or isinstance(v, (int, np.integer)):
        return out + f_varint(3, int(v)) + f_varint(20, 2)
    if isinstance(v, float):
        return out + f_float(2, v) + f_varint(20, 1)
    if isinstance(v, str):
        return out + f_bytes(4, v.encode()) + f_varint(20, 3)
    if isinstance(v, np.ndarray):
        return out + f_bytes(5, tensor("", v)) + f_varint(20, 4)
    v = list(v)
    if v and isinstance(v[0], float):
        return out + b"".join(f_float(7, x) for x in v) + f_varint(20, 6)
    return out + f_ints(8, v) + f_varint(20, 7)


def node(op: str, inputs, outputs, name: str = "", **attrs) -> bytes:
    out = b"".join(f_str(1, i) for i in inputs) + b"".join(f_str(2, o) for o in outputs)
    if name:
        out += f_str(3, name)
    out += f_str(4, op)
    for k, v in attrs.items():
        out += f_bytes(5, attr(k, v))
    return out


def value_info(name: str, shape, elem=FLOAT) -> bytes:
    dims = b""
    for d in shape:
        dims += f_bytes(1, f_varint(1, d) if isinstance(d, int) else f_str(2, str(d)))
    tt = f_varint(1, elem) + f_bytes(2, dims)
    return f_str(1, name) + f_bytes(2, f_bytes(1, tt))


def model(nodes, inits, inputs, outputs, opset=13, ir_version=7, producer="dw-tests") -> bytes:
    g = b"".join(f_bytes(1, n) for n in nodes) + f_str(2, "graph")
    g += b"".join(f_bytes(5, t) for t in inits)
    g += b"".join(f_bytes(11, v) for v in inputs) + b"".join(f_bytes(12, v) for v in outputs)
    return (f_varint(1, ir_version) + f_str(2, producer) + f_bytes(7, g) +
            f_bytes(8, f_str(1, "") + f_varint(2, opset)))


# ---------------------------------------------------------------------------
# exporters from the graph IR (Graph.to_dict() + initializer access)
# ---------------------------------------------------------------------------
def _conv_attrs(op):
    return dict(kernel_shape=op["kernel_shape"], strides=op["strides"], pads=op["pads"],
                dilations=op["dilations"], group=op["group"])


def export_float_nchw(g) -> bytes:
    """The F32 NCHW graph (before any pass) as ONNX, opset 13: Split sizes
    as an int64 input, Resize with roi / scales inputs."""
    d = g.to_dict()
    t = d["tensors"]
    nodes, inits, vin, _ = _float_parts(g)
    vout = [value_info(n, t[n]["dims"]) for n in d["outputs"]]
    return model(nodes, inits, vin, vout)


def export_qdq(g) -> bytes:
    """A u8 QDQ graph of this repository (NHWC, after quantize_qdq) as a QDQ
    ONNX model in NCHW: every u8 tensor becomes its float producer followed
    by QuantizeLinear -> DequantizeLinear; QLinearConv becomes
    DequantizeLinear(int8 OIHW weights, per-channel, axis 0) + Conv (+ int32
    bias through DequantizeLinear); the table after it becomes Sigmoid + Mul;
    QLinearAdd an Add; the convs that stayed fp16 plain Convs with their f16
    weights widened to f32."""
    d = g.to_dict()
    t = d["tensors"]
    nodes, inits = [], []
    qdone = set()

    def nchw(dims):
        return [dims[0], dims[3], dims[1], dims[2]] if len(dims) == 4 else list(dims)

    def u8(name):  # the dequantized (float) name of a u8 tensor
        return name + ".deq"

    def emit_qdq(name):
        if name in qdone:
            return
        qdone.add(name)
        ti = t[name]
        s, z = name + ".q_scale", name + ".q_zp"
        inits.append(tensor(s, np.array(ti["scale"], np.float32)))
        inits.append(tensor(z, np.array(ti["zp"], np.uint8)))
        nodes.append(node("QuantizeLinear", [name + ".pre_q", s, z], [name + ".u8"], name + ".quantize"))
        nodes.append(node("DequantizeLinear", [name + ".u8", s, z], [u8(name)], name + ".dequantize"))

    def src(name):  # the float tensor a consumer reads
        return u8(name) if t[name]["dtype"] == 3 else name

    def dst(name):  # the float tensor a producer writes (then Q/DQ for u8)
        return name + ".pre_q" if t[name]["dtype"] == 3 else name

    for op in d["ops"]:
        ty, ins, outs = op["type"], op["inputs"], op["outputs"]
        if ty == "QuantizeLinear":  # f16 -> u8: the float tensor is the input itself
            nodes.append(node("Identity", [src(ins[0])], [dst(outs[0])], op["name"]))
        elif ty == "DequantizeLinear":
            nodes.append(node("Identity", [src(ins[0])], [outs[0]], op["name"]))
        elif ty in ("QLinearConv", "QGemm"):
            w = ins[1]
            wd = t[w]["dims"]
            wq = g.initializer(w, np.int8, tuple(wd))
            ws = np.array(t[w]["ch_scales"], np.float32)
            wn = w + ".q"
            sn = w + ".scales"
            if ty == "QLinearConv":
                inits.append(tensor(wn, np.ascontiguousarray(wq.transpose(3, 2, 0, 1))))
                nodes.append(node("DequantizeLinear", [wn, sn], [w + ".w"], w + ".dequantize", axis=0))
            else:
                inits.append(tensor(wn, np.ascontiguousarray(wq.reshape(wd[2], wd[3]))))
                nodes.append(node("DequantizeLinear", [wn, sn], [w + ".w"], w + ".dequantize", axis=1))
            inits.append(tensor(sn, ws))
            cins = [src(ins[0]), w + ".w"]
            if len(ins) > 2 and ins[2]:
                b = ins[2]
                xs = t[ins[0]]["scale"]
                inits.append(tensor(b + ".q", g.initializer(b, np.int32, (wd[3],))))
                inits.append(tensor(b + ".scales", (np.float32(xs) * ws).astype(np.float32)))
                nodes.append(node("DequantizeLinear", [b + ".q", b + ".scales"], [b + ".b"], b + ".dequantize",
                                  axis=0))
                cins.append(b + ".b")
            if ty == "QLinearConv":
                nodes.append(node("Conv", cins, [dst(outs[0])], op["name"], **_conv_attrs(op)))
            else:
                nodes.append(node("Gemm", cins, [dst(outs[0])], op["name"]))
        elif ty == "QLinearLUT":
            sg = outs[0] + ".sigmoid"
            nodes.append(node("Sigmoid", [src(ins[0])], [sg], op["name"] + "_sigmoid"))
            nodes.append(node("Mul", [src(ins[0]), sg], [dst(outs[0])], op["name"]))
        elif ty == "QLinearAdd":
            nodes.append(node("Add", [src(i) for i in ins], [dst(outs[0])], op["name"]))
        elif ty == "Conv":  # a conv kept fp16: f32 weights in the model
            w = ins[1]
            wd = t[w]["dims"]
            wf = g.initializer(w, np.float16, tuple(wd)).astype(np.float32).transpose(3, 2, 0, 1)
            inits.append(tensor(w, np.ascontiguousarray(wf)))
            cins = [src(ins[0]), w]
            if len(ins) > 2 and ins[2]:
                inits.append(tensor(ins[2], g.initializer(ins[2], np.float16, (wd[3],)).astype(np.float32)))
                cins.append(ins[2])
            nodes.append(node("Conv", cins, [dst(outs[0])], op["name"], **_conv_attrs(op)))
        elif ty in ("MaxPool", "Resize", "Concat", "Split"):
            o = dict(op)
            if ty == "Concat" or ty == "Split":
                o["axis"] = 1 if op["axis"] == 3 else op["axis"]
            fins = [src(i) for i in ins]
            fouts = [dst(x) for x in outs]
            if ty == "MaxPool":
                nodes.append(node(ty, fins, fouts, op["name"], kernel_shape=op["kernel_shape"],
                                  strides=op["strides"], pads=op["pads"]))
            elif ty == "Resize":
                x = nchw(t[ins[0]]["dims"])
                sc = op["name"] + ".scales"
                inits.append(tensor(sc, np.array([1, 1, op["out_h"] / x[2], op["out_w"] / x[3]], np.float32)))
                nodes.append(node(ty, [fins[0], "", sc], fouts, op["name"], mode="nearest"))
            elif ty == "Concat":
                nodes.append(node(ty, fins, fouts, op["name"], axis=o["axis"]))
            else:
                sp = op["name"] + ".split"
                inits.append(tensor(sp, np.array(op["split_sizes"], np.int64)))
                nodes.append(node(ty, [fins[0], sp], fouts, op["name"], axis=o["axis"]))
        else:
            raise NotImplementedError(ty)
        for o_ in outs:
            if t[o_]["dtype"] == 3:
                emit_qdq(o_)
    vin = [value_info(n, nchw(t[n]["dims"])) for n in d["inputs"]]
    vout = [value_info(src(n), nchw(t[n]["dims"])) for n in d["outputs"]]
    return model(nodes, inits, vin, vout)


# ---------------------------------------------------------------------------
# the exported YOLOv8 detect tail (ultralytics Detect in export mode)
# ---------------------------------------------------------------------------
def make_anchors(level_hw, strides):
    """Anchor points (cell centres, row-major per level) as [1, 2, A] and the
    per-anchor stride as [1, A] (ultralytics make_anchors, offset 0.5)."""
    pts, st = [], []
    for (h, w), s in zip(level_hw, strides):
        sy, sx = np.meshgrid(np.arange(h, dtype=np.float32) + 0.5, np.arange(w, dtype=np.float32) + 0.5,
                             indexing="ij")
        pts.append(np.stack([sx.ravel(), sy.ravel()], 0))
        st.append(np.full(h * w, s, np.float32))
    return np.concatenate(pts, 1)[None].astype(np.float32), np.concatenate(st)[None].astype(np.float32)


def exported_tail(levels, level_dims, strides, nc=80, reg_max=16, shape_ops=False, out="output0"):
    """Nodes and initializers of the exported tail over the per-level head
    outputs `levels` (NCHW [b, 4 reg_max + nc, h, w]):
      Reshape [b, no, h*w] per level -> Concat axis 2 -> Split [4R, nc] axis 1;
      DFL: Reshape [b, 4, R, A] -> Transpose (0, 2, 1, 3) -> Softmax axis 1 ->
        Conv 1x1 (R -> 1, weights 0..R-1) -> Reshape [b, 4, A];
      dist2bbox: Slice lt / rb -> anchors - lt, anchors + rb -> (x1y1 + x2y2) / 2,
        x2y2 - x1y1 -> Concat axis 1 -> Mul strides;
      Sigmoid of the classes; Concat axis 1 -> [b, 4 + nc, A].
    With shape_ops the Reshape shapes are computed as unsimplified exports do
    (Shape -> Gather -> Unsqueeze -> Concat of constants)."""
    b = level_dims[0][0]
    no = 4 * reg_max + nc
    hw = [(d[2], d[3]) for d in level_dims]
    A = sum(h * w for h, w in hw)
    nodes, inits = [], []

    def const(name, arr):
        inits.append(tensor(name, np.asarray(arr)))
        return name

    def shape_of(tag, src, rest):
        """the shape [b] + rest, from Shape(src)[0] when shape_ops"""
        if not shape_ops:
            return const(f"{tag}.shape", np.array([b] + list(rest), np.int64))
        nodes.append(node("Shape", [src], [f"{tag}.s"], f"{tag}.shape_op"))
        nodes.append(node("Gather", [f"{tag}.s", const(f"{tag}.i0", np.array(0, np.int64))], [f"{tag}.b"],
                          f"{tag}.gather", axis=0))
        nodes.append(node("Unsqueeze", [f"{tag}.b", const(f"{tag}.ax", np.array([0], np.int64))], [f"{tag}.b1"],
                          f"{tag}.unsqueeze"))
        nodes.append(node("Concat", [f"{tag}.b1", const(f"{tag}.rest", np.array(rest, np.int64))], [f"{tag}.shape"],
                          f"{tag}.concat", axis=0))
        return f"{tag}.shape"

    flat = []
    for i, (x, (h, w)) in enumerate(zip(levels, hw)):
        sh = shape_of(f"tail.r{i}", x, [no, -1])
        nodes.append(node("Reshape", [x, sh], [f"tail.r{i}"], f"tail.reshape{i}"))
        flat.append(f"tail.r{i}")
    nodes.append(node("Concat", flat, ["tail.cat"], "tail.concat", axis=2))
    nodes.append(node("Split", ["tail.cat", const("tail.split", np.array([4 * reg_max, nc], np.int64))],
                      ["tail.box", "tail.cls"], "tail.split_op", axis=1))
    sh = shape_of("tail.dfl", "tail.box", [4, reg_max, A])
    nodes.append(node("Reshape", ["tail.box", sh], ["tail.dfl.r"], "tail.dfl.reshape"))
    nodes.append(node("Transpose", ["tail.dfl.r"], ["tail.dfl.t"], "tail.dfl.transpose", perm=[0, 2, 1, 3]))
    nodes.append(node("Softmax", ["tail.dfl.t"], ["tail.dfl.p"], "tail.dfl.softmax", axis=1))
    dflw = const("tail.dfl.w", np.arange(reg_max, dtype=np.float32).reshape(1, reg_max, 1, 1))
    nodes.append(node("Conv", ["tail.dfl.p", dflw], ["tail.dfl.c"], "tail.dfl.conv", kernel_shape=[1, 1]))
    sh = shape_of("tail.dist", "tail.dfl.c", [4, A])
    nodes.append(node("Reshape", ["tail.dfl.c", sh], ["tail.dist"], "tail.dist.reshape"))
    ax1 = const("tail.ax1", np.array([1], np.int64))
    nodes.append(node("Slice", ["tail.dist", const("tail.s0", np.array([0], np.int64)),
                                const("tail.e2", np.array([2], np.int64)), ax1], ["tail.lt"], "tail.slice_lt"))
    nodes.append(node("Slice", ["tail.dist", const("tail.s2", np.array([2], np.int64)),
                                const("tail.e4", np.array([4], np.int64)), ax1], ["tail.rb"], "tail.slice_rb"))
    anchors, stv = make_anchors(hw, strides)
    const("tail.anchors", anchors)
    const("tail.strides", stv)
    nodes.append(node("Sub", ["tail.anchors", "tail.lt"], ["tail.x1y1"], "tail.sub1"))
    nodes.append(node("Add", ["tail.anchors", "tail.rb"], ["tail.x2y2"], "tail.add1"))
    nodes.append(node("Add", ["tail.x1y1", "tail.x2y2"], ["tail.csum"], "tail.add2"))
    nodes.append(node("Div", ["tail.csum", const("tail.two", np.array(2.0, np.float32))], ["tail.cxy"], "tail.div"))
    nodes.append(node("Sub", ["tail.x2y2", "tail.x1y1"], ["tail.wh"], "tail.sub2"))
    nodes.append(node("Concat", ["tail.cxy", "tail.wh"], ["tail.dbox0"], "tail.concat_box", axis=1))
    nodes.append(node("Mul", ["tail.dbox0", "tail.strides"], ["tail.dbox"], "tail.mul_stride"))
    nodes.append(node("Sigmoid", ["tail.cls"], ["tail.scores"], "tail.sigmoid"))
    nodes.append(node("Concat", ["tail.dbox", "tail.scores"], [out], "tail.concat_out", axis=1))
    return nodes, inits, (b, 4 + nc, A)


def export_float_nchw_with_tail(g, strides=(8, 16, 32), shape_ops=False, opset=17, keep_heads=False) -> bytes:
    """export_float_nchw of the YOLOv8n-shaped graph with the exported detect
    tail after its three per-level outputs: the model's output is
    output0 [b, 84, A] (and the three head tensors after it with keep_heads)."""
    d = g.to_dict()
    t = d["tensors"]
    nodes, inits, vin, _ = _float_parts(g)
    heads = d["outputs"]
    tn, ti, odims = exported_tail(heads, [t[h]["dims"] for h in heads], strides, shape_ops=shape_ops)
    vout = [value_info("output0", list(odims))]
    if keep_heads:
        vout += [value_info(h, t[h]["dims"]) for h in heads]
    return model(nodes + tn, inits + ti, vin, vout, opset=opset)


def _float_parts(g):
    """The node, initializer and input lists export_float_nchw writes."""
    d = g.to_dict()
    t = d["tensors"]
    nodes, inits = [], []
    for name, ti in t.items():
        if ti["init"]:
            inits.append(tensor(name, g.initializer(name, np.float32, tuple(ti["dims"]))))
    for op in d["ops"]:
        ty, ins, outs = op["type"], op["inputs"], op["outputs"]
        if ty == "Conv":
            nodes.append(node("Conv", ins, outs, op["name"], **_conv_attrs(op)))
        elif ty == "BatchNormalization":
            nodes.append(node(ty, ins, outs, op["name"], epsilon=float(op["epsilon"])))
        elif ty in ("Sigmoid", "Mul", "Add", "Relu"):
            nodes.append(node(ty, ins, outs, op["name"]))
        elif ty == "Concat":
            nodes.append(node(ty, ins, outs, op["name"], axis=op["axis"]))
        elif ty == "Split":
            sp = op["name"] + ".split"
            inits.append(tensor(sp, np.array(op["split_sizes"], np.int64)))
            nodes.append(node(ty, [ins[0], sp], outs, op["name"], axis=op["axis"]))
        elif ty == "MaxPool":
            nodes.append(node(ty, ins, outs, op["name"], kernel_shape=op["kernel_shape"], strides=op["strides"],
                              pads=op["pads"]))
        elif ty == "Resize":
            x = t[ins[0]]["dims"]
            sc = op["name"] + ".scales"
            inits.append(tensor(sc, np.array([1, 1, op["out_h"] / x[2], op["out_w"] / x[3]], np.float32)))
            nodes.append(node(ty, [ins[0], "", sc], outs, op["name"], mode="nearest",
                              coordinate_transformation_mode="asymmetric", nearest_mode="floor"))
        else:
            raise NotImplementedError(ty)
    vin = [value_info(n, t[n]["dims"]) for n in d["inputs"]]
    return nodes, inits, vin, None


def tail_reference_nchw(heads, strides=(8, 16, 32), nc=80, reg_max=16):
    """The exported tail's meaning, in f64 numpy on NCHW head outputs (an
    independent statement of the ONNX graph above)."""
    b = heads[0].shape[0]
    x = np.concatenate([h.astype(np.float64).reshape(b, h.shape[1], -1) for h in heads], 2)
    box, cls = x[:, :4 * reg_max], x[:, 4 * reg_max:]
    d = box.reshape(b, 4, reg_max, -1)
    e = np.exp(d - d.max(axis=2, keepdims=True))
    p = e / e.sum(axis=2, keepdims=True)
    dist = (p * np.arange(reg_max).reshape(1, 1, reg_max, 1)).sum(axis=2)
    anchors, stv = make_anchors([h.shape[2:] for h in heads], strides)
    a = anchors.astype(np.float64)
    x1y1, x2y2 = a - dist[:, :2], a + dist[:, 2:]
    dbox = np.concatenate([(x1y1 + x2y2) / 2, x2y2 - x1y1], 1) * stv.astype(np.float64)
    return np.concatenate([dbox, 1 / (1 + np.exp(-cls))], 1)
