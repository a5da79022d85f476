"""The reference's own graph forms on the HIP runtime, against the oracle's
CpuGraph:

* the symmetric INT8 form QuantizedGraphCompiler emits (quantize.rs:73-368):
  Quantize, Conv writing t with Requantize reading the unwritten "t_i32" and
  writing t again (quantize.rs:205-223), Relu, AddQuantized, MaxPool, a
  Concat / Split whose axis is still NCHW-numbered after
  convert_nchw_to_nhwc (graph.rs:248-290), Dequantize -- run as built and
  after fusion pass 3 (Conv2dRequantReluI8, fusion.rs:192-334); bit-exact;
* Clip, Softmax and Reshape (vulkan_runtime.rs:549-584);
* Conv + Relu after fusion pass 1, which keeps the ReLU;
* one backend shared by two host threads.
"""
import threading

import numpy as np
import pytest

import oracle
from oracle.cpu_graph import CpuGraph
from dragonwing_edge_rs_amd import ops, synth
from dragonwing_edge_rs_amd.graph import GRAPH_F16, GRAPH_F32, GRAPH_I8, Graph, HipGraphRuntime


def oracle_run(g, inputs):
    cg = CpuGraph(g.to_dict(), g.initializer)
    for k, v in inputs.items():
        cg.set_input(k, v)
    return cg.run()


def ref_int8_graph(n=2, h=20, w=20, seed=7, i32_output=False):
    """The reference's INT8 graph form, restated: per-output-channel weight
    scales absmax/127 and q = clamp(round(w / s)) (quantize.rs:344-368),
    activation scales absmax/127, requant scale s_in * mean(s_w) / s_out
    (quantize.rs:205-223, :307-325), AddQuantized ratios (quantize.rs:263-288)."""
    r = synth.Rng(synth.seed_for(seed))
    g = Graph(GRAPH_I8)

    def qweights(name, kh, kw, ci, co):
        wf = r.uniform((kh, kw, ci, co), -1.0, 1.0).astype(np.float32)
        s = np.abs(wf).reshape(-1, co).max(axis=0) / np.float32(127.0)
        q = np.clip(np.round(wf * (np.float32(1.0) / s)), -128, 127).astype(np.int8)
        g.add_initializer(name, q, "i8")
        return float(np.mean(s, dtype=np.float32))

    s_x, s1, s2, s_add, s3 = 1.0 / 127, 0.09, 0.11, 0.13, 0.07
    g.add_tensor("x", (n, h, w, 16), "f32")
    g.add_tensor("xq", (n, h, w, 16), "i8")
    g.add_op("quant", "Quantize", ["x"], ["xq"], scale=s_x)

    def conv_requant(name, src, ci, co, k, s_in, s_out, relu, stride=1):
        ws = qweights(name + ".w", k, k, ci, co)
        shape_in = sizes[src]
        ho = (shape_in[1] + 2 * (k // 2) - k) // stride + 1
        wo = (shape_in[2] + 2 * (k // 2) - k) // stride + 1
        out = (n, ho, wo, co)
        g.add_tensor(name, out, "i8")
        g.add_tensor(name + "_i32", out, "i32")
        g.add_op(name, "Conv", [src, name + ".w"], [name], kernel_shape=(k, k), strides=(stride, stride),
                 pads=(k // 2,) * 4)
        g.add_op(name + "_requant", "Requantize", [name + "_i32"], [name], scale=s_in * ws / s_out)
        sizes[name] = out
        last = name
        if relu:
            g.add_tensor(name + ".relu", out, "i8")
            g.add_op(name + ".relu", "Relu", [name], [name + ".relu"])
            sizes[name + ".relu"] = out
            last = name + ".relu"
        return last

    sizes = {"xq": (n, h, w, 16)}
    a1 = conv_requant("c1", "xq", 16, 32, 3, s_x, s1, True)
    c2 = conv_requant("c2", a1, 32, 32, 3, s1, s2, False)
    g.add_tensor("sum", (n, h, w, 32), "i8")
    g.add_op("add", "AddQuantized", [a1, c2], ["sum"], scale_a_over_out=s1 / s_add, scale_b_over_out=s2 / s_add)
    g.add_tensor("pool", (n, h // 2, w // 2, 32), "i8")
    g.add_op("pool", "MaxPool", ["sum"], ["pool"], kernel_shape=(2, 2), strides=(2, 2))
    sizes["pool"] = (n, h // 2, w // 2, 32)
    c3 = conv_requant("c3", "pool", 32, 16, 1, s_add, s3, True)
    g.add_tensor("cat", (n, h // 2, w // 2, 48), "i8")
    g.add_op("cat", "Concat", ["pool", c3], ["cat"], axis=1)  # NCHW channel axis left by the pass
    g.add_tensor("u", (n, h // 2, w // 2, 16), "i8")
    g.add_tensor("v", (n, h // 2, w // 2, 32), "i8")
    g.add_op("split", "Split", ["cat"], ["u", "v"], axis=1, split_sizes=(16, 32))
    g.add_tensor("out", (n, h // 2, w // 2, 32), "f32")
    g.add_op("dequant", "Dequantize", ["v"], ["out"], scale=s_add)
    g.add_tensor("u_f", (n, h // 2, w // 2, 16), "f32")
    g.add_op("dequant_u", "Dequantize", ["u"], ["u_f"], scale=s3)
    g.add_tensor("clip", (n, h // 2, w // 2, 16), "f32")
    g.add_op("clip", "Clip", ["u_f"], ["clip"], clip_min=0.0, clip_max=6.0 * s3 * 10)
    g.add_tensor("rows", (n * (h // 2) * (w // 2), 16), "f32")
    g.add_op("reshape", "Reshape", ["clip"], ["rows"])
    g.add_tensor("prob", (n * (h // 2) * (w // 2), 16), "f32")
    g.add_op("softmax", "Softmax", ["rows"], ["prob"], axis=1)
    outs = ["out", "prob"] + (["c2_i32"] if i32_output else [])
    g.set_io(["x"], outs)
    x = r.uniform((n, h, w, 16), -1.0, 1.0).astype(np.float32)
    return g, x, outs


def outputs_of(rt, g, outs):
    d = g.to_dict()["tensors"]
    np_dt = {0: np.float32, 2: np.int8, 4: np.int32}
    return {o: rt.get_output_bytes(o).view(np_dt[d[o]["dtype"]]).reshape(d[o]["dims"]) for o in outs}


def check_ref_graph(backend, g, x, outs, exact_softmax=False):
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32("x", x)
    rt.run()
    got = outputs_of(rt, g, outs)
    ref = oracle_run(g, {"x": x})
    for o in outs:
        if o == "prob" and not exact_softmax:
            # softmax's exp is the device's: a few ulps from the host's
            np.testing.assert_allclose(got[o], ref[o], rtol=1e-5, atol=1e-7, err_msg=o)
        else:
            np.testing.assert_array_equal(got[o], ref[o], err_msg=o)
    assert len(np.unique(got["out"])) > 20  # not degenerate
    return rt


@pytest.mark.gpu
def test_reference_int8_graph_as_built(backend):
    g, x, outs = ref_int8_graph()
    rt = check_ref_graph(backend, g, x, outs)
    kinds = [L["kernel"].split("_")[0] for L in rt.launches()]
    assert kinds.count("igemm") == 3  # each Conv + Requantize (+ Relu) is one launch


@pytest.mark.gpu
def test_reference_int8_graph_after_fusion_pass3(backend):
    g, x, outs = ref_int8_graph()
    g.apply_fusion_passes()
    types = [op["type"] for op in g.to_dict()["ops"]]
    assert types.count("Conv2dRequantReluI8") == 3 and "Requantize" not in types
    check_ref_graph(backend, g, x, outs)


@pytest.mark.gpu
def test_reference_int8_graph_int32_accumulator_output(backend):
    # c2's accumulator is also a graph output: the conv writes int32 and the
    # Requantize runs as its own kernel
    g, x, outs = ref_int8_graph(i32_output=True)
    rt = check_ref_graph(backend, g, x, outs)
    assert "elementwise" in [L["kernel"] for L in rt.launches()]


@pytest.mark.gpu
@pytest.mark.parametrize("tile", ["32,4,-2", "32,2,-1", "32,4,2", "16,1,0"])
def test_reference_int8_graph_every_kernel_variant(backend, monkeypatch, tile):
    # the s8 operand path and the reference requantize epilogue on the
    # row-tile, streamed, persistent and staged kernels
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    g, x, outs = ref_int8_graph(n=1, h=40, w=40)
    check_ref_graph(backend, g, x, outs)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [GRAPH_F32, GRAPH_F16])
def test_conv_relu_fused_by_pass1(backend, dtype):
    # fusion pass 1 leaves one Conv writing the Relu's output; the ReLU is
    # kept (has_relu) and results equal the unfused graph's oracle run.
    r = synth.Rng(synth.seed_for(31))
    et = "f32" if dtype == GRAPH_F32 else "f16"
    def build():
        g = Graph(dtype)
        g.add_tensor("x", (2, 12, 12, 16), et)
        w = r.uniform((3, 3, 16, 24), -0.5, 0.5)
        b = r.uniform((24,), -0.2, 0.2)
        if et == "f16":
            g.add_initializer("w", synth.f16_bits(w), "f16")
            g.add_initializer("b", synth.f16_bits(b), "f16")
        else:
            g.add_initializer("w", w.astype(np.float32))
            g.add_initializer("b", b.astype(np.float32))
        g.add_tensor("c", (2, 12, 12, 24), et)
        g.add_tensor("y", (2, 12, 12, 24), et)
        g.add_op("conv", "Conv", ["x", "w", "b"], ["c"], kernel_shape=(3, 3), pads=(1, 1, 1, 1))
        g.add_op("relu", "Relu", ["c"], ["y"])
        g.set_io(["x"], ["y"])
        return g
    g0 = build()
    r = synth.Rng(synth.seed_for(31))
    g1 = build()
    assert g1.apply_fusion_passes() == 1
    x = synth.Rng(synth.seed_for(32)).uniform((2, 12, 12, 16), -1.0, 1.0).astype(np.float32)
    xin = x if et == "f32" else synth.f16_bits(x)
    ref = oracle_run(g0, {"x": xin})["y"]
    rt = HipGraphRuntime(g1, backend)
    rt.set_input_f32("x", x)
    rt.run()
    got = rt.get_output_bytes("y").view(np.float32 if et == "f32" else np.uint16).reshape(ref.shape)
    if et == "f32":
        np.testing.assert_array_equal(got, ref)
    else:  # the fp16 MFMA conv accumulates in another order
        err = np.max(np.abs(oracle.f16_to_f32(got) - oracle.f16_to_f32(ref))) / np.max(np.abs(oracle.f16_to_f32(ref)))
        assert err <= 1e-2
    assert np.all(got.view(np.int16 if et == "f16" else np.int32) >= 0)  # no negative results survive


@pytest.mark.gpu
def test_clip_softmax_f16(backend):
    r = synth.Rng(synth.seed_for(33))
    g = Graph(GRAPH_F16)
    g.add_tensor("x", (4, 3, 5, 16), "f16")
    g.add_tensor("c", (4, 3, 5, 16), "f16")
    g.add_tensor("s", (4, 3, 5, 16), "f16")
    g.add_op("clip", "Clip", ["x"], ["c"], clip_min=-1.5, clip_max=2.25)
    g.add_op("soft", "Softmax", ["c"], ["s"], axis=-1)
    g.set_io(["x"], ["c", "s"])
    x = synth.f16_bits(r.normal((4, 3, 5, 16), 0.0, 2.0))
    x.ravel()[::37] = np.uint16(0x7E00)  # NaN passes through Clip
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", x)
    rt.run()
    ref = oracle_run(g, {"x": x})
    c = rt.get_output_bytes("c").view(np.uint16).reshape(x.shape)
    np.testing.assert_array_equal(c, ref["c"])
    s = oracle.f16_to_f32(rt.get_output_bytes("s").view(np.uint16).reshape(x.shape))
    sr = oracle.f16_to_f32(ref["s"])
    np.testing.assert_allclose(s, sr, rtol=1e-2, atol=1e-3, equal_nan=True)


@pytest.mark.gpu
def test_backend_shared_by_two_threads(backend):
    # Two host threads run QLinearConv ops of different sizes on one backend
    # (the packed-weight and scale workspaces grow and are reused under
    # both); every result must equal the oracle's.
    cases = [synth.qlinearconv_case(40 + t, n=1, h=12 + 8 * t, w=12 + 8 * t, c_in=32 * (t + 1), c_out=64 * (t + 1))
             for t in range(2)]
    refs = []
    for c in cases:
        refs.append(oracle.qlinearconv_u8s8(c["x"], c["w"], c["bias"], (1, 1), (1, 1), c["x_scale"], c["x_zp"],
                                            c["w_scales"], c["y_scale"], c["y_zp"]))
    errors = []

    def worker(t):
        try:
            c = cases[t]
            n, h, w, ci = c["x"].shape
            co = c["w"].shape[3]
            bx, bw, bb = backend.from_numpy(c["x"]), backend.from_numpy(c["w"]), backend.from_numpy(c["bias"])
            by = backend.alloc(n * h * w * co)
            for it in range(40):
                ops.qlinearconv_u8s8(backend, bx, bw, bb, by, n, h, w, ci, co, 3, 3, 1, 1, 1, 1, c["x_scale"],
                                     c["x_zp"], c["w_scales"], c["y_scale"], c["y_zp"])
                if it % 8 == 7:
                    got = backend.to_numpy(by, np.uint8, (n, h, w, co))
                    if not np.array_equal(got, refs[t]):
                        errors.append(f"thread {t} iteration {it}: {(got != refs[t]).sum()} bytes differ")
                        return
        except Exception as e:  # reported below
            errors.append(f"thread {t}: {e!r}")

    th = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in th), "a worker thread did not finish"
    assert not errors, errors


def test_reference_int8_graph_oracle_forms_agree():
    # CPU: the oracle runs the reference's INT8 form as built and after
    # fusion pass 3 to the same bytes, and its INT8 conv chain equals an
    # int64 brute force with requantize's clamp-then-round-half-away.
    g, x, outs = ref_int8_graph(n=1, h=8, w=8)
    a = oracle_run(g, {"x": x})
    g2, _, _ = ref_int8_graph(n=1, h=8, w=8)
    g2.apply_fusion_passes()
    b = oracle_run(g2, {"x": x})
    for o in outs:
        np.testing.assert_array_equal(a[o], b[o])
    # brute force of c1 (3x3 pad 1, then requant + relu)
    d = g.to_dict()
    xq = a["xq"].astype(np.int64)
    w1 = g.initializer("c1.w", np.int8, (3, 3, 16, 32)).astype(np.int64)
    xp = np.pad(xq, ((0, 0), (1, 1), (1, 1), (0, 0)))
    acc = np.zeros((1, 8, 8, 32), np.int64)
    for kh in range(3):
        for kw in range(3):
            acc += np.einsum("nhwc,cd->nhwd", xp[:, kh:kh + 8, kw:kw + 8, :], w1[kh, kw])
    scale = next(op["scale"] for op in d["ops"] if op["name"] == "c1_requant")
    f = np.clip(acc.astype(np.float32) * np.float32(scale), -128, 127)
    q = (np.sign(f) * np.floor(np.abs(f).astype(np.float64) + 0.5)).astype(np.int8)  # half away from zero
    np.testing.assert_array_equal(a["c1.relu"], np.maximum(q, 0))


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1, 3, 5])
def test_maxpool_cascade_radius(backend, k):
    # Three chained k x k stride-1 MaxPools with pads k // 2 run as one
    # cascade launch; k = 1 (radius 0, each pool the identity) included.
    r = synth.Rng(synth.seed_for(50 + k))
    g = Graph(GRAPH_F16)
    shape = (2, 9, 11, 16)
    for t in ("x", "p1", "p2", "p3"):
        g.add_tensor(t, shape, "f16")
    for i, (a, b) in enumerate((("x", "p1"), ("p1", "p2"), ("p2", "p3"))):
        g.add_op(f"pool{i}", "MaxPool", [a], [b], kernel_shape=(k, k), strides=(1, 1), pads=(k // 2,) * 4)
    g.set_io(["x"], ["p1", "p2", "p3"])
    x = synth.f16_bits(r.normal(shape, 0.0, 1.0))
    rt = HipGraphRuntime(g, backend)
    assert [L["kernel"] for L in rt.launches()] == ["maxpool_cascade3"]
    rt.set_input_bytes("x", x)
    rt.run()
    ref = oracle_run(g, {"x": x})
    for t in ("p1", "p2", "p3"):
        np.testing.assert_array_equal(rt.get_output_bytes(t).view(np.uint16).reshape(shape), ref[t], err_msg=t)
    if k == 1:
        np.testing.assert_array_equal(ref["p3"], x)
