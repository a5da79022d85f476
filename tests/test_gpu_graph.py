"""GPU parity of the graph runtime (HipGraphRuntime) on YOLOv8n-shaped
graphs against the oracle's CpuGraphRuntime restatement.

* fp16 graph: max|gpu - ref| <= 1e-2 * max|ref| per detect output (the MFMA
  convs accumulate in another order than the CPU);
* f32 graph (the calibration graph): <= 1e-3 relative (only expf may differ);
* int8 (u8 QDQ) graph, two plans:
  - exact (DW_RT_EXACT_U8_F16_CONV): bit-exact, including the fp16 stem and
    the fp16 head 1x1 convs, at a small size and at the full 640x640
    batch-32 workload (every image of the batch against a batch-1 oracle
    run, on the graph built from the oracle Calibrator's ranges);
  - default (the head's u8 -> f16 1x1 convs on the fp16 matrix cores): every
    INT8 part bit-exact -- checked on the head convs' u8 inputs, the last
    tensors the INT8 layers write -- and the fp16 head outputs within 1e-2,
    at a small size and on every image of the graph the benchmark times.
"""
import numpy as np
import pytest

import oracle
from oracle.cpu_graph import CpuGraph
from oracle.cpu_graph import calibrate as calibrate_oracle
from dragonwing_edge_rs_amd import synth, yolo
from dragonwing_edge_rs_amd.graph import HipGraphRuntime

pytestmark = pytest.mark.gpu


def oracle_run(g, inputs: dict):
    cg = CpuGraph(g.to_dict(), g.initializer)
    for k, v in inputs.items():
        cg.set_input(k, v)
    return cg.run()


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def gpu_outputs(rt, info, dtype=np.uint16):
    return [rt.get_output_bytes(o).view(dtype).reshape(s) for o, s in zip(info["outputs"], info["out_shapes"])]


def head_inputs(g):
    """The u8 tensors the fp16 head convs read (through DequantizeLinear):
    the last tensors the INT8 layers write."""
    d = g.to_dict()
    prod = {o: op for op in d["ops"] for o in op["outputs"]}
    heads = []
    for op in d["ops"]:
        src = prod.get(op["inputs"][0]) if op["type"] == "Conv" else None
        if src is not None and src["type"] == "DequantizeLinear":
            heads.append(src["inputs"][0])
    return heads


def expose_head_inputs(g, info):
    """Makes the head convs' u8 inputs graph outputs too (after the detect
    outputs); returns their names and shapes."""
    heads = head_inputs(g)
    assert len(heads) == 6, heads
    g.set_io([info["input"]], list(info["outputs"]) + heads)
    dims = g.to_dict()["tensors"]
    return [(h, tuple(dims[h]["dims"])) for h in heads]


def mfma_head_outputs(rt, info, heads):
    """The head inputs and the detect outputs of a run, downloaded once."""
    return {h: rt.get_output_bytes(h).reshape(shp) for h, shp in heads}, gpu_outputs(rt, info)


def check_mfma_head(got, info, heads, ref, img=None):
    """Default plan: the head inputs (INT8 parts) bit-exact, the fp16 head
    outputs within 1e-2 of each output's largest magnitude.  got: the run's
    tensors (mfma_head_outputs); ref: the oracle's tensors (for image img of
    the batch when img is given)."""
    sl = slice(None) if img is None else slice(img, img + 1)
    got_heads, got_outs = got
    for h, shp in heads:
        np.testing.assert_array_equal(got_heads[h][sl], ref[h], err_msg=h)
    worst = 0.0
    for o, gv in zip(info["outputs"], got_outs):
        e = rel_err(oracle.f16_to_f32(gv[sl]), oracle.f16_to_f32(ref[o]))
        worst = max(worst, e)
        assert e <= 1e-2, (o, e)
    return worst


def test_f16_graph_small_vs_oracle(backend):
    g, info = yolo.f16_graph(batch=2, size=96)
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        e = rel_err(oracle.f16_to_f32(gv), oracle.f16_to_f32(ref[o]))
        print(f"{o}: rel err {e:.2e}")
        assert e <= 1e-2


def test_f32_graph_small_vs_oracle(backend):
    g, info = yolo.build_yolov8n(batch=1, size=64)
    g.fold_batchnorm()
    g.convert_nchw_to_nhwc()
    x = yolo.input_images(1, 64)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    ref = oracle_run(g, {info["input"]: x})
    for o, s in zip(info["outputs"], info["out_shapes"]):
        got = rt.get_output_bytes(o).view(np.float32).reshape(s)
        assert rel_err(got, ref[o]) <= 1e-3


@pytest.fixture(scope="module")
def int8_small(backend):
    return yolo.int8_graph(backend, batch=2, size=96, calib=yolo.calibration_images(16, 96))


def test_int8_graph_small_bit_exact(backend, int8_small):
    g, info = int8_small
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        assert gv.shape == ref[o].shape
        np.testing.assert_array_equal(gv, ref[o], err_msg=o)
    # the result is not degenerate
    assert len(np.unique(got[0])) > 100


def test_int8_graph_small_mfma_head(backend):
    # Default plan: the six head 1x1 convs (u8 in, f16 out) on the fp16
    # matrix cores; the INT8 parts bit-exact, the head outputs within 1e-2.
    g, info = yolo.int8_graph(backend, batch=2, size=96, calib=yolo.calibration_images(16, 96))
    heads = expose_head_inputs(g, info)
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend)
    kinds = [L["kernel"] for L in rt.launches()]
    assert kinds.count("conv1x1_u8_f16") == 6 and kinds.count("stem_pad_u8") == 1, kinds
    rt.set_input_f32(info["input"], x)
    rt.run()
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    worst = check_mfma_head(mfma_head_outputs(rt, info, heads), info, heads, ref)
    print(f"head outputs: worst rel err {worst:.2e}")
    # the exact plan of the same graph gives the oracle's bytes
    rt_x = HipGraphRuntime(g, backend, exact_u8_f16=True)
    kinds = [L["kernel"] for L in rt_x.launches()]
    assert kinds.count("direct_conv") == 6 and kinds.count("stem_pad_u8") == 1, kinds
    rt_x.set_input_f32(info["input"], x)
    rt_x.run()
    for o, gv in zip(info["outputs"], gpu_outputs(rt_x, info)):
        np.testing.assert_array_equal(gv, ref[o], err_msg=o)


def test_int8_graph_corrected_quotient_bit_exact(backend, int8_small, monkeypatch):
    # The fp16 stem's u8 epilogue divides by the output scale as a product
    # with the reciprocal, plus an FMA correction unless the host proved the
    # plain product exact for every f16 value; the corrected form gives the
    # same bytes.
    monkeypatch.setenv("DW_QUANT_CORRECTED", "1")
    g, info = int8_small
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    rt.set_input_f32(info["input"], x)
    rt.run()
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], gpu_outputs(rt, info)):
        np.testing.assert_array_equal(gv, ref[o], err_msg=o)


@pytest.mark.parametrize("tile", ["16,4,3", "32,2,1", "64,4,2", "128,2,5"])
def test_int8_graph_persistent_tiles_bit_exact(backend, int8_small, monkeypatch, tile):
    # Every convolution whose K fits the persistent kernel runs on it with
    # this tile (requantize, activation table and residual epilogues).
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    g, info = int8_small
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    if tile == "16,4,3":
        assert any(l["kernel"].endswith("_t3") for l in rt.launches())
    rt.set_input_f32(info["input"], x)
    rt.run()
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], gpu_outputs(rt, info)):
        np.testing.assert_array_equal(gv, ref[o], err_msg=f"{o} tile {tile}")


@pytest.mark.parametrize("tile", ["256,4,-3", "128,4,-3", "64,4,-3"])
def test_int8_graph_wide_tiles_bit_exact(backend, monkeypatch, tile):
    # Every layer with c_in a multiple of 128 on the wide-tile kernel
    # (requantize, table and table + residual epilogues).
    g, info = yolo.int8_graph(backend, batch=2, size=160, calib=yolo.calibration_images(4, 160))
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    x = yolo.input_images(2, 160)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    assert sum(L["kernel"].endswith("_wide") for L in rt.launches()) >= 4
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=f"{o} tile {tile}")


@pytest.mark.parametrize("tile", ["256,4,-3", "128,4,-3", "64,4,-3"])
def test_f16_graph_wide_tiles_identical(backend, monkeypatch, tile):
    # Every fp16 layer with c_in a multiple of 64 on the wide-tile kernel
    # (with and without the residual add): the same bytes as the staged
    # kernel's, which the other graph tests hold to the oracle.
    g, info = yolo.f16_graph(batch=2, size=160)
    x = yolo.input_images(2, 160)
    monkeypatch.setenv("DW_IGEMM_TILE", "16,4")
    rt0 = HipGraphRuntime(g, backend)
    rt0.set_input_f32(info["input"], x)
    rt0.run()
    ref = gpu_outputs(rt0, info)
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    rt = HipGraphRuntime(g, backend)
    assert sum(L["kernel"].endswith("_wide") for L in rt.launches()) >= 4
    rt.set_input_f32(info["input"], x)
    rt.run()
    for o, a, b in zip(info["outputs"], ref, gpu_outputs(rt, info)):
        np.testing.assert_array_equal(b, a, err_msg=f"{o} tile {tile}")


@pytest.mark.parametrize("tile", ["128,1,-1", "64,2,-1", "32,4,-1"])
def test_int8_graph_streamed_tiles_bit_exact(backend, int8_small, monkeypatch, tile):
    # Every layer with two or more k-steps on the streamed-weight kernel
    # (all four int8 epilogues: requantize, table, table + residual).
    g, info = int8_small
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    assert any(L["kernel"].endswith("_st") for L in rt.launches())
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=f"{o} tile {tile}")


def test_int8_graph_row_tiles_bit_exact(backend, monkeypatch):
    # 320x320 input: the 80- and 40-wide stride-1 3x3 layers (C2f bottlenecks,
    # P3 detect heads) take the row-tile kernel, with the table and the
    # table + residual epilogues.
    g, info = yolo.int8_graph(backend, batch=1, size=320, calib=yolo.calibration_images(4, 320))
    monkeypatch.setenv("DW_IGEMM_TILE", "16,4,-2")
    x = yolo.input_images(1, 320)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    assert sum(L["kernel"].endswith("_rows") for L in rt.launches()) >= 10
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=o)


@pytest.mark.parametrize("tile", ["16,10,-4", "32,10,-4", "64,5,-4", "64,10,-4", "80,10,-4", "16,10,-5", "32,10,-5",
                                  "64,10,-5", "80,10,-5"])
def test_int8_graph_band_tiles_bit_exact(backend, monkeypatch, tile):
    # 320x320 input: the stride-1 3x3 layers the band-tile kernel accepts for
    # the forced channel tile and band height (C2f bottlenecks with the table
    # and table + residual epilogues, detect heads), exact plan: every output
    # bit-exact against the oracle.
    g, info = yolo.int8_graph(backend, batch=1, size=320, calib=yolo.calibration_images(4, 320))
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    monkeypatch.setenv("DW_PAIR", "0")
    x = yolo.input_images(1, 320)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    bands = [L["ops"] for L in rt.launches() if "_band" in L["kernel"]]
    print(f"tile {tile}: {len(bands)} band launches", flush=True)
    assert len(bands) >= 2, bands
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=f"{o} tile {tile}")


@pytest.mark.parametrize("rows", [None, "1", "2", "5"])
def test_int8_graph_c2f_bit_exact(backend, monkeypatch, rows):
    # 320x320 input: the one-bottleneck C2f blocks with 16 or 32 hidden
    # channels (b2 at 80x80 with the shortcut, the neck's P3 block at 40x40
    # without) each in one launch, the block's intermediates in LDS; the
    # tuner's band height and forced small ones (bands of 1 and 2 rows: the
    # halo rows reach past the band's neighbours), exact plan: every output
    # bit-exact against the oracle.
    g, info = yolo.int8_graph(backend, batch=1, size=320, calib=yolo.calibration_images(4, 320))
    monkeypatch.setenv("DW_C2F", "1")
    monkeypatch.setenv("DW_PAIR", "0")
    if rows:
        monkeypatch.setenv("DW_C2F_ROWS", rows)
    x = yolo.input_images(1, 320)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    fused = [L["ops"].split("+")[0] for L in rt.launches() if L["kernel"].startswith("igemm_i8_c2f")]
    print(f"rows {rows}: fused C2f blocks {fused}", flush=True)
    assert {"b2.cv1", "n15.cv1"} <= set(fused), fused
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=f"{o} rows {rows}")


def test_int8_benchmark_graph_c2f_same_bytes(backend, monkeypatch):
    # The benchmark's batch-32 640x640 graph with its one-bottleneck C2f
    # blocks fused (DW_C2F=1) and not (DW_C2F=0): the same bytes.
    from dragonwing_edge_rs_amd import workloads
    g, _, _, _, info = workloads.yolov8n_int8(backend)
    x = yolo.input_images(32, 640)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DW_C2F", mode)
        rt = HipGraphRuntime(g, backend)
        fused = [L["ops"].split("+")[0] for L in rt.launches() if L["kernel"].startswith("igemm_i8_c2f")]
        print(f"DW_C2F={mode}: fused {fused}", flush=True)
        assert (len(fused) >= 2) == (mode == "1"), fused
        rt.set_input_f32(info["input"], x)
        rt.run()
        outs[mode] = gpu_outputs(rt, info)
    for o, a, b in zip(info["outputs"], outs["0"], outs["1"]):
        np.testing.assert_array_equal(a, b, err_msg=o)


@pytest.mark.parametrize("tile", [None, "64,4", "32,4,-2"])
def test_int8_graph_resize_fused_bit_exact(backend, monkeypatch, tile):
    # 320x320 input: the neck's two nearest 2x upsamples written by the
    # epilogues of the convs that produce their inputs (the upsampled bytes
    # stored at each output pixel's four pixels of the concat slice), with
    # the tuner's tiles and forced staged / row tiles; exact plan, every
    # output bit-exact against the oracle.
    g, info = yolo.int8_graph(backend, batch=1, size=320, calib=yolo.calibration_images(4, 320))
    monkeypatch.setenv("DW_RESIZE_FUSE", "1")
    if tile:
        monkeypatch.setenv("DW_IGEMM_TILE", tile)
    x = yolo.input_images(1, 320)
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    ks = [L["kernel"] for L in rt.launches()]
    print(f"tile {tile}: resize launches {ks.count('resize_nearest')}", flush=True)
    assert "resize_nearest" not in ks, ks
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=f"{o} tile {tile}")


def test_int8_benchmark_graph_resize_fused_same_bytes(backend, monkeypatch):
    # The benchmark's batch-32 640x640 graph with its upsamples folded into
    # their producers (DW_RESIZE_FUSE=1) and as separate launches (=0): the
    # same bytes.
    from dragonwing_edge_rs_amd import workloads
    g, _, _, _, info = workloads.yolov8n_int8(backend)
    x = yolo.input_images(32, 640)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DW_RESIZE_FUSE", mode)
        rt = HipGraphRuntime(g, backend)
        n = sum(L["kernel"] == "resize_nearest" for L in rt.launches())
        print(f"DW_RESIZE_FUSE={mode}: {n} resize launches", flush=True)
        assert n == (2 if mode == "0" else 0), n
        rt.set_input_f32(info["input"], x)
        rt.run()
        outs[mode] = gpu_outputs(rt, info)
    for o, a, b in zip(info["outputs"], outs["0"], outs["1"]):
        np.testing.assert_array_equal(a, b, err_msg=o)


@pytest.mark.parametrize("size,batch", [(320, 1), (640, 32)])
def test_f16_graph_resize_fused_same_bytes(backend, monkeypatch, size, batch):
    # The fp16 graph's upsamples written by the epilogues of the convs that
    # produce their inputs (DW_RESIZE_FUSE=1) and as separate launches (=0):
    # the same f16 values.
    g, info = yolo.f16_graph(batch=batch, size=size)
    x = yolo.input_images(batch, size)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DW_RESIZE_FUSE", mode)
        rt = HipGraphRuntime(g, backend)
        n = sum(L["kernel"] == "resize_nearest" for L in rt.launches())
        print(f"{size} DW_RESIZE_FUSE={mode}: {n} resize launches", flush=True)
        assert n == (2 if mode == "0" else 0), n
        rt.set_input_f32(info["input"], x)
        rt.run()
        outs[mode] = gpu_outputs(rt, info)
    for o, a, b in zip(info["outputs"], outs["0"], outs["1"]):
        np.testing.assert_array_equal(a, b, err_msg=o)


@pytest.mark.parametrize("tile", ["64,10,-4", "80,10,-4"])
def test_int8_graph_band_head_same_bytes(backend, monkeypatch, tile):
    # The detect heads' fused u8 -> f16 1x1 on the band-tile kernel: the same
    # bytes as the separate 1x1 launches.
    g, info = yolo.int8_graph(backend, batch=2, size=320, calib=yolo.calibration_images(4, 320))
    x = yolo.input_images(2, 320)
    monkeypatch.setenv("DW_PAIR", "0")
    monkeypatch.setenv("DW_HEAD_FUSE", "0")
    rt0 = HipGraphRuntime(g, backend)
    rt0.set_input_f32(info["input"], x)
    rt0.run()
    ref = gpu_outputs(rt0, info)
    monkeypatch.setenv("DW_HEAD_FUSE", "1")
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    rt = HipGraphRuntime(g, backend)
    heads = [L["kernel"] for L in rt.launches() if L["kernel"].endswith("_head")]
    print(f"tile {tile}: heads {heads}", flush=True)
    assert any("_band" in k for k in heads), heads
    rt.set_input_f32(info["input"], x)
    rt.run()
    for o, a, b in zip(info["outputs"], ref, gpu_outputs(rt, info)):
        np.testing.assert_array_equal(b, a, err_msg=f"{o} tile {tile}")


@pytest.mark.parametrize("plant_subnormal_weight", [False, True])
@pytest.mark.parametrize("stride", [1, 2])
@pytest.mark.parametrize("shape", [(2, 23, 29, 48), (1, 9, 83, 64), (3, 17, 40, 192)])
def test_depthwise_graph_bit_exact(backend, plant_subnormal_weight, stride, shape):
    # Depthwise conv + bias without activation, exact plan: bit-exact, on
    # the path that feeds the f16 weights straight into the fma and (one
    # weight planted subnormal) on the path that widens them as the
    # reference does; the inputs carry subnormals too.  The default plan
    # (the band kernel where it applies) within the fp16 tolerance.
    from dragonwing_edge_rs_amd.graph import Graph, GRAPH_F16
    r = synth.Rng(synth.seed_for(900 + stride + shape[2]))
    n, h, w, c = shape
    x = synth.f16_bits(r.normal((n, h, w, c), 0.0, 1.0))
    x.ravel()[::997] = np.uint16(0x0003)  # subnormal inputs scattered over the tensor
    wt = synth.f16_bits(r.normal((3, 3, 1, c), 0.0, 0.3))
    if plant_subnormal_weight:
        wt[1, 2, 0, 5] = np.uint16(0x8011)
    b = synth.f16_bits(r.normal((c,), 0.0, 0.1))
    ho, wo = oracle.out_hw(h, w, 3, 3, stride, stride, 1, 1)
    g = Graph(GRAPH_F16)
    g.add_tensor("x", x.shape, "f16")
    g.add_initializer("w", wt, "f16")
    g.add_initializer("b", b, "f16")
    g.add_tensor("y", (n, ho, wo, c), "f16")
    g.add_op("dw", "Conv", ["x", "w", "b"], ["y"], kernel_shape=(3, 3), strides=(stride, stride),
             pads=(1, 1, 1, 1), group=c)
    g.set_io(["x"], ["y"])
    rt = HipGraphRuntime(g, backend, exact_f16_dw=True)
    rt.set_input_bytes("x", x)
    rt.run()
    got = rt.get_output_bytes("y").view(np.uint16).reshape(n, ho, wo, c)
    ref = oracle_run(g, {"x": x})["y"]
    np.testing.assert_array_equal(got, ref)
    # the default plan's band kernel (stride 1, c % 64 == 0) within the fp16 tolerance
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", x)
    rt.run()
    got = rt.get_output_bytes("y").view(np.uint16).reshape(n, ho, wo, c)
    assert rel_err(oracle.f16_to_f32(got), oracle.f16_to_f32(ref)) <= 1e-2


def test_int8_graph_capture_replays_match_eager(backend, int8_small):
    g, info = int8_small
    x = yolo.input_images(2, 96)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    eager = gpu_outputs(rt, info)
    rt.enable_capture(True)
    for i in range(4):
        rt.set_input_f32(info["input"], x if i % 2 == 0 else np.zeros_like(x))
        rt.run()
        outs = gpu_outputs(rt, info)
        if i % 2 == 0:
            for a, b in zip(outs, eager):
                np.testing.assert_array_equal(a, b)
        backend.synchronize()


def test_int8_graph_streams_match_one_stream(backend, int8_small, monkeypatch):
    # Independent launches run on several streams (parallel branches of the
    # captured graph); the results must equal the one-stream schedule's, on
    # every replay, eagerly and captured.
    g, info = int8_small
    x = yolo.input_images(2, 96)
    monkeypatch.setenv("DW_GRAPH_STREAMS", "1")
    rt1 = HipGraphRuntime(g, backend)
    monkeypatch.setenv("DW_GRAPH_STREAMS", "4")
    rt4 = HipGraphRuntime(g, backend)
    rt1.set_input_f32(info["input"], x)
    rt1.run()
    ref = gpu_outputs(rt1, info)
    for capture in (False, True):
        rt4.enable_capture(capture)
        for i in range(3):
            rt4.set_input_f32(info["input"], x if i % 2 == 0 else np.zeros_like(x))
            rt4.run()
            outs = gpu_outputs(rt4, info)
            if i % 2 == 0:
                for a, b in zip(outs, ref):
                    np.testing.assert_array_equal(a, b)
            backend.synchronize()


def test_activation_reuse_matches_unshared_storage(backend, int8_small, monkeypatch):
    # Storage whose lifetimes do not overlap shares the activation arena;
    # on four streams (independent detect-head branches run concurrently,
    # so reused bytes must wait for their last readers) and captured, the
    # outputs equal those of a runtime where every tensor has its own bytes.
    g, info = int8_small
    x = yolo.input_images(2, 96)
    monkeypatch.setenv("DW_ACT_REUSE", "0")
    ref_rt = HipGraphRuntime(g, backend)
    monkeypatch.setenv("DW_ACT_REUSE", "1")
    monkeypatch.setenv("DW_GRAPH_STREAMS", "4")
    rt = HipGraphRuntime(g, backend)
    arena, unshared = rt.activation_bytes()
    ref_arena, ref_unshared = ref_rt.activation_bytes()
    assert ref_arena == ref_unshared == unshared
    assert arena < 0.6 * unshared, (arena, unshared)
    ref_rt.set_input_f32(info["input"], x)
    ref_rt.run()
    ref = gpu_outputs(ref_rt, info)
    for capture in (False, True):
        rt.enable_capture(capture)
        for i in range(3):
            rt.set_input_f32(info["input"], x if i % 2 == 0 else np.zeros_like(x))
            rt.run()
            outs = gpu_outputs(rt, info)
            if i % 2 == 0:
                for a, b in zip(outs, ref):
                    np.testing.assert_array_equal(a, b)
            backend.synchronize()


def test_run_unbatched_and_io(backend, int8_small, monkeypatch):
    g, info = int8_small
    rt = HipGraphRuntime(g, backend)
    assert rt.inputs() == [(info["input"], (2, 96, 96, 3))]
    assert [n for n, _ in rt.outputs()] == info["outputs"]
    assert [s for _, s in rt.outputs()] == [tuple(s) for s in info["out_shapes"]]
    x = yolo.input_images(2, 96)
    rt.set_input_f32(info["input"], x)
    rt.run()
    ref = gpu_outputs(rt, info)
    rt.set_input_f32(info["input"], np.zeros_like(x))
    rt.run()
    rt.set_input_f32(info["input"], x)
    monkeypatch.setenv("DW_TRACE", "1")
    rt.run_unbatched()
    for a, b in zip(gpu_outputs(rt, info), ref):
        np.testing.assert_array_equal(a, b)


def test_int8_graph_launch_plan(backend, int8_small):
    g, info = int8_small
    rt = HipGraphRuntime(g, backend)
    ls = rt.launches()
    kinds = {}
    for L in ls:
        kinds[L["kernel"].split("_")[0]] = kinds.get(L["kernel"].split("_")[0], 0) + 1
    # 56 int8 MFMA convs (each with its table / residual fused; two chained
    # 3x3 convs in one launch, or a whole one-bottleneck C2f block's four,
    # where the tuner finds that faster), the fp16 stem as an exact-order conv,
    # the six fp16 head 1x1 convs on the fp16 matrix cores (each in its own
    # launch or inside its 3x3's, "_head"), one SPPF cascade, two resizes
    # (each in its own launch or written by the conv before it, "_up"), no
    # copies or elementwise; a detect scale's box0 and cls0 as one GEMM
    # ("_sib") where the tuner finds that faster.
    pairs = sum(L["kernel"].startswith("igemm_i8_pair") for L in ls)
    blocks = sum(L["kernel"].startswith("igemm_i8_c2f") for L in ls)
    heads = sum(L["kernel"].endswith("_head") for L in ls)
    sibs = sum(L["kernel"].endswith("_sib") for L in ls)
    assert kinds.get("igemm") + pairs + 3 * blocks + sibs == 56, (pairs, blocks, sibs, kinds)
    assert kinds.get("direct", 0) + kinds.get("stem", 0) == 1 and kinds.get("conv1x1", 0) + heads == 6, kinds
    ups = sum(L["kernel"].endswith("_up") for L in ls)
    assert kinds.get("maxpool") == 1 and kinds.get("resize", 0) + ups == 2, kinds
    assert "copy" not in kinds and "elementwise" not in kinds, kinds
    ms = rt.run_profiled()
    assert len(ms) == len(ls) and np.all(ms > 0)


def test_int8_graph_pairs_bit_exact(backend, monkeypatch):
    # At 320x320 the C2f bottlenecks of the 80x80 (16 channels), 40x40 (32
    # channels, with and without the shortcut) and 20x20 (64 channels) maps,
    # and the first two 3x3 convs of the stride-8 detect head's box branch
    # (64 channels, 40x40), run as chained pairs, the intermediate in LDS:
    # bit-exact against the oracle, and the same bytes as the unchained
    # launches.
    g, info = yolo.int8_graph(backend, batch=2, size=320, calib=yolo.calibration_images(4, 320))
    x = yolo.input_images(2, 320)
    monkeypatch.setenv("DW_PAIR", "1")  # every candidate pair, whatever the timing
    monkeypatch.setenv("DW_C2F", "0")  # the one-bottleneck blocks as pairs too
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    pairs = sorted(L["kernel"].replace("_w16", "") for L in rt.launches() if L["kernel"].startswith("igemm_i8_pair"))
    assert pairs == ["igemm_i8_pair_c16"] + ["igemm_i8_pair_c32"] * 3 + ["igemm_i8_pair_c64"] * 5, pairs
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=o)
    # every band height (rows per workgroup; heights invalid for a pair
    # leave its choice as it is), and the unchained launches
    for rows in ("1", "2", "4", "5", "8"):
        monkeypatch.setenv("DW_PAIR_ROWS", rows)
        rtr = HipGraphRuntime(g, backend, exact_u8_f16=True)
        rtr.set_input_f32(info["input"], x)
        rtr.run()
        for o, gv, gr in zip(info["outputs"], got, gpu_outputs(rtr, info)):
            np.testing.assert_array_equal(gv, gr, err_msg=f"{o} rows {rows}")
    monkeypatch.delenv("DW_PAIR_ROWS")
    # the 16-wave form of every pair
    monkeypatch.setenv("DW_PAIR_WAVES", "16")
    rtw = HipGraphRuntime(g, backend, exact_u8_f16=True)
    assert all(L["kernel"].endswith("_w16") for L in rtw.launches() if L["kernel"].startswith("igemm_i8_pair"))
    rtw.set_input_f32(info["input"], x)
    rtw.run()
    for o, gv, gw in zip(info["outputs"], got, gpu_outputs(rtw, info)):
        np.testing.assert_array_equal(gv, gw, err_msg=f"{o} 16 waves")
    monkeypatch.delenv("DW_PAIR_WAVES")
    monkeypatch.setenv("DW_PAIR", "0")
    rt0 = HipGraphRuntime(g, backend, exact_u8_f16=True)
    assert not any(L["kernel"].startswith("igemm_i8_pair") for L in rt0.launches())
    rt0.set_input_f32(info["input"], x)
    rt0.run()
    for o, gv, g0 in zip(info["outputs"], got, gpu_outputs(rt0, info)):
        np.testing.assert_array_equal(gv, g0, err_msg=o)


@pytest.mark.parametrize("size,batch", [(320, 2), (640, 32)])
def test_int8_graph_head_fusion_same_bytes(backend, monkeypatch, size, batch):
    # The detect heads' u8 -> f16 1x1 convs fused into the epilogue of the
    # 3x3 QLinearConv before them (the u8 results regrouped in LDS and fed to
    # the fp16 matrix cores): the same bytes as the separate 1x1 launches
    # (whose outputs test_int8_benchmark_graph checks against the oracle),
    # at 320x320 and on the benchmark's batch-32 640x640 graph.
    if size == 640:
        from dragonwing_edge_rs_amd import workloads
        g, _, _, _, info = workloads.yolov8n_int8(backend)
    else:
        g, info = yolo.int8_graph(backend, batch=batch, size=size, calib=yolo.calibration_images(4, size))
    x = yolo.input_images(batch, size)
    monkeypatch.setenv("DW_PAIR", "0")
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DW_HEAD_FUSE", mode)
        rt = HipGraphRuntime(g, backend)
        fused = [L["kernel"] for L in rt.launches() if L["kernel"].endswith("_head")]
        assert len(fused) == (6 if mode == "1" else 0), fused
        assert sum(L["kernel"] == "conv1x1_u8_f16" for L in rt.launches()) == (0 if mode == "1" else 6)
        rt.set_input_f32(info["input"], x)
        rt.run()
        outs[mode] = gpu_outputs(rt, info)
    for o, a, b in zip(info["outputs"], outs["0"], outs["1"]):
        np.testing.assert_array_equal(a, b, err_msg=o)


def gpu_ranges(backend, batch, size, images):
    from dragonwing_edge_rs_amd.graph import calibrate
    gc, info = yolo.calibration_graph(batch, size)
    calibrate(backend, gc, info["input"], images)
    return {n: tuple(t["range"]) for n, t in gc.to_dict()["tensors"].items() if "range" in t}, info


def oracle_ranges(batch, size, images):
    gc, info = yolo.calibration_graph(batch, size)
    return calibrate_oracle(gc.to_dict(), gc.initializer, info["input"], images)


def compare_ranges(gr, orr, input_name):
    """GPU calibration ranges against the oracle Calibrator's: the same
    tensors (the GPU also records the graph input).  The f32 graph's convs
    and adds are bit-exact, but its sigmoid's expf is the device's, a few
    ulps from the host libm's on some inputs, and every tensor downstream of
    the first sigmoid can carry that into its extremes.  So: the tensors no
    sigmoid feeds (the stem conv's output) must be identical; the others are
    counted, and the worst relative difference of a scale (absmax / 127) is
    returned with the count."""
    assert set(gr) - set(orr) == {input_name}, set(gr) ^ set(orr)
    same, worst = 0, 0.0
    for n, (lo, hi) in orr.items():
        glo, ghi = gr[n]
        if (glo, ghi) == (np.float32(lo), np.float32(hi)):
            same += 1
        so, sg = oracle.scale_from_range(lo, hi), oracle.scale_from_range(glo, ghi)
        worst = max(worst, abs(float(sg) - float(so)) / float(so))
    assert gr["b0.bn_out"] == tuple(np.float32(v) for v in orr["b0.bn_out"])  # no expf upstream
    return same, len(orr), worst


def test_calibration_matches_oracle_small(backend):
    imgs = yolo.calibration_images(4, 96)
    gr, info = gpu_ranges(backend, 2, 96, imgs)
    orr = oracle_ranges(2, 96, imgs)
    same, total, worst = compare_ranges(gr, orr, info["input"])
    print(f"calibration 96x96, 4 images: {same} of {total} ranges identical, worst scale difference {worst:.2e}")
    assert worst <= 1e-5


def check_int8_batch_bit_exact(g, info, x, backend, graph1, monkeypatch):
    """Runs the batch-32 u8 graph g on the GPU (exact plan, every candidate
    pair of chained 3x3 convs in one launch) and compares every image of the
    batch with the oracle's CpuGraph run on the same graph at batch 1."""
    monkeypatch.setenv("DW_PAIR", "1")
    monkeypatch.setenv("DW_C2F", "0")  # the one-bottleneck blocks as pairs too
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    # the eight C2f bottlenecks of 16, 32 and 64 channels (with and without
    # the shortcut) and the stride-8 head's first two box convs run as
    # chained pairs
    pairs = [L["kernel"].replace("_w16", "") for L in rt.launches() if L["kernel"].startswith("igemm_i8_pair")]
    assert sorted(pairs) == sorted(["igemm_i8_pair_c16"] + ["igemm_i8_pair_c32"] * 3 + ["igemm_i8_pair_c64"] * 5), pairs
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    g1, info1 = graph1
    for img in range(x.shape[0]):
        ref = oracle_run(g1, {info1["input"]: synth.f16_bits(x[img:img + 1])})
        for o, gv in zip(info["outputs"], got):
            np.testing.assert_array_equal(gv[img:img + 1], ref[o], err_msg=f"{o} image {img}")
        if img % 8 == 7:
            print(f"images 0..{img} bit-exact", flush=True)
    print(f"all {x.shape[0]} images bit-exact on all three detect outputs", flush=True)


def test_int8_graph_full_workload_bit_exact(backend, monkeypatch):
    # The headline workload end to end: the oracle Calibrator over the 16
    # seeded calibration images at 640x640 fixes every activation scale; the
    # GPU's calibration of the same images agrees with it (counted and
    # bounded); the u8 graph built from the oracle's ranges runs at batch 32
    # on the GPU and matches the oracle's CpuGraph bit for bit on every image
    # of the batch.
    imgs = yolo.calibration_images(16, 640)
    orr = oracle_ranges(1, 640, imgs)
    gr, info0 = gpu_ranges(backend, 16, 640, imgs)
    same, total, worst = compare_ranges(gr, orr, info0["input"])
    print(f"calibration 640x640, 16 images: {same} of {total} ranges identical, "
          f"worst scale difference {worst:.2e}", flush=True)
    assert worst <= 1e-5
    g, info = yolo.int8_graph_from_ranges(orr, batch=32, size=640)
    x = yolo.input_images(32, 640)
    check_int8_batch_bit_exact(g, info, x, backend, yolo.int8_graph_from_ranges(orr, batch=1, size=640), monkeypatch)


def test_int8_benchmark_graph(backend):
    # The graph and plan the benchmark times (workloads.yolov8n_int8: scales
    # from the GPU's own calibration of the 16 seeded images; the head's
    # u8 -> f16 1x1 convs on the fp16 matrix cores), all 32 images of the
    # benchmark's input batch against the oracle's CpuGraph on that graph:
    # the INT8 parts (the head convs' u8 inputs) bit-exact, the fp16 head
    # outputs within 1e-2.
    from dragonwing_edge_rs_amd import workloads

    g, inputs, outs, work, info = workloads.yolov8n_int8(backend)
    x = yolo.input_images(32, 640)
    np.testing.assert_array_equal(inputs[info["input"]], synth.f16_bits(x))
    heads = expose_head_inputs(g, info)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    # the same passes over the same ranges at batch 1, with the same outputs
    g1, info1 = yolo.int8_graph_from_ranges(info["ranges"], batch=1, size=640)
    expose_head_inputs(g1, info1)
    worst = 0.0
    got = mfma_head_outputs(rt, info, heads)
    for img in range(32):
        ref = oracle_run(g1, {info1["input"]: synth.f16_bits(x[img:img + 1])})
        worst = max(worst, check_mfma_head(got, info, heads, ref, img))
        if img % 8 == 7:
            print(f"images 0..{img} checked", flush=True)
    print(f"all 32 images: INT8 parts bit-exact, head outputs worst rel err {worst:.2e}", flush=True)


def test_f16_graph_full_workload_vs_oracle(backend):
    # cfg4: the fp16 YOLOv8n-shaped graph at batch 32, 640x640; every image
    # against the oracle's CpuGraph at batch 1, within 1e-2 of each detect
    # output's largest magnitude (the MFMA convs accumulate in another order
    # than the CPU's fma chain).
    g, info = yolo.f16_graph(batch=32, size=640)
    x = yolo.input_images(32, 640)
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    g1, info1 = yolo.f16_graph(batch=1, size=640)
    worst = 0.0
    for img in range(32):
        ref = oracle_run(g1, {info1["input"]: synth.f16_bits(x[img:img + 1])})
        for o, gv in zip(info["outputs"], got):
            e = rel_err(oracle.f16_to_f32(gv[img:img + 1]), oracle.f16_to_f32(ref[o]))
            worst = max(worst, e)
            assert e <= 1e-2, (o, img, e)
        if img % 8 == 7:
            print(f"images 0..{img} within tolerance", flush=True)
    print(f"all 32 images within tolerance, worst rel err {worst:.2e}", flush=True)


def test_single_op_graphs(backend):
    """The single-op workloads expressed as graphs: QLinearConv (bit-exact),
    depthwise fp16 + SiLU (fp16 tolerance), fp32 conv + ReLU (bit-exact)."""
    from dragonwing_edge_rs_amd import workloads

    g, inputs, outs, work, c = workloads.qlinearconv()
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", inputs["x"])
    rt.run()
    got = rt.get_output_bytes("y").reshape(32, 40, 40, 256)
    ref = oracle.qlinearconv_u8s8(c["x"], c["w"], c["bias"], (2, 2), (1, 1), c["x_scale"], c["x_zp"],
                                  c["w_scales"], c["y_scale"], c["y_zp"])
    np.testing.assert_array_equal(got, ref)
    assert [L["kernel"].split("_")[0] for L in rt.launches()] == ["igemm"]

    g, inputs, outs, work, (x, w, b) = workloads.dwconv()
    ref = oracle_run(g, {"x": x})["out"]
    # the default plan: the packed-f16 band kernel, within the fp16 tolerance
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", inputs["x"])
    rt.run()
    got = rt.get_output_bytes("out").view(np.uint16).reshape(x.shape)
    e = rel_err(oracle.f16_to_f32(got), oracle.f16_to_f32(ref))
    print(f"depthwise band kernel: rel err {e:.2e}, {np.mean(got != ref):.3f} of the outputs differ")
    assert e <= 1e-2
    assert [L["kernel"].split("_u")[0] for L in rt.launches()] == ["dwconv3_tile"]
    # the exact plan: the reference's f32 chain, last-bit flips of the f16 sigmoid only
    rt = HipGraphRuntime(g, backend, exact_f16_dw=True)
    rt.set_input_bytes("x", inputs["x"])
    rt.run()
    got = rt.get_output_bytes("out").view(np.uint16).reshape(x.shape)
    assert rel_err(oracle.f16_to_f32(got), oracle.f16_to_f32(ref)) <= 1e-2
    assert np.mean(got != ref) < 1e-3
    assert [L["kernel"] for L in rt.launches()] == ["dwconv_f16"]

    g, inputs, outs, work, (x, w, b) = workloads.conv_f32()
    rt = HipGraphRuntime(g, backend)
    rt.set_input_f32("x", x)
    rt.run()
    got = rt.get_output_bytes("out").view(np.float32).reshape(1, 56, 56, 64)
    np.testing.assert_array_equal(got, oracle.relu_f32(oracle.bias_add_f32(oracle.conv2d_f32_nhwc(x, w, (1, 1), (1, 1)), b)))
    assert [L["kernel"] for L in rt.launches()] == ["direct_conv"]


@pytest.mark.parametrize("ci,k,s,p,co,n,h,w,act", [
    (3, 3, 2, 1, 16, 2, 64, 64, "silu"),    # the YOLO stem, whole 16-pixel blocks per row
    (3, 3, 2, 1, 48, 3, 37, 29, "silu"),    # ragged rows, an odd last band
    (3, 3, 2, 1, 64, 1, 21, 70, "none"),
    (1, 5, 1, 2, 32, 2, 19, 23, "silu"),    # K = 25
    (2, 3, 1, 1, 16, 1, 9, 33, "none"),     # K = 18
    (3, 1, 1, 0, 64, 2, 17, 16, "silu"),    # K = 3
])
def test_f16_stem_mfma_vs_oracle(backend, ci, k, s, p, co, n, h, w, act):
    # the fp16 graphs' convs whose whole K fits one fp16 k-step run on the
    # fp16 matrix cores (stem_f16_mfma): within 1e-2 of the oracle's output's
    # largest magnitude, every shape class of the kernel (rows of whole or
    # ragged 16-pixel blocks, a last band of one row, 1..4 channel blocks)
    from dragonwing_edge_rs_amd.graph import Graph, GRAPH_F16

    r = np.random.default_rng(1000 + ci * 100 + k * 10 + co)
    x = synth.f16_bits(r.normal(0.0, 1.0, (n, h, w, ci)))
    wt = synth.f16_bits(r.normal(0.0, (1.0 / (k * k * ci)) ** 0.5, (k, k, ci, co)))
    b = synth.f16_bits(r.normal(0.0, 0.1, (co,)))
    ho, wo = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    g = Graph(GRAPH_F16)
    g.add_tensor("x", x.shape, "f16")
    g.add_initializer("w", wt, "f16")
    g.add_initializer("b", b, "f16")
    out = "y" if act == "none" else "out"
    for t in ("y", "sg", "out") if act != "none" else ("y",):
        g.add_tensor(t, (n, ho, wo, co), "f16")
    g.add_op("conv", "Conv", ["x", "w", "b"], ["y"], kernel_shape=(k, k), strides=(s, s), pads=(p, p, p, p))
    if act != "none":
        g.add_op("sig", "Sigmoid", ["y"], ["sg"])
        g.add_op("mul", "Mul", ["y", "sg"], ["out"])
    g.set_io(["x"], [out])
    ref = oracle_run(g, {"x": x})[out]
    rt = HipGraphRuntime(g, backend)
    rt.set_input_bytes("x", x)
    rt.run()
    assert [L["kernel"] for L in rt.launches()] == ["stem_f16_mfma"]
    got = rt.get_output_bytes(out).view(np.uint16).reshape(n, ho, wo, co)
    e = rel_err(oracle.f16_to_f32(got), oracle.f16_to_f32(ref))
    print(f"stem {ci}x{k}x{k}/{s} -> {co} at {n}x{h}x{w}: rel err {e:.2e}", flush=True)
    assert e <= 1e-2
    # the same input as NCHW f32 planes, read by the stem itself: the same bytes
    xn = np.ascontiguousarray(synth.f16_value(x).transpose(0, 3, 1, 2))
    rt.set_input_nchw_f32("x", xn)
    rt.run()
    assert rt.get_output_bytes(out).view(np.uint16).reshape(n, ho, wo, co).tobytes() == got.tobytes()


def test_int8_graph_siblings_bit_exact(backend, int8_small, monkeypatch):
    # each detect scale's box0 and cls0 QLinearConvs (same input) as one GEMM
    # over both channel sets, every channel tile writing its own conv's
    # output with its own table: forced for all three scales, the oracle's
    # bytes, and the bytes of the unfused plan
    g, info = int8_small
    x = yolo.input_images(2, 96)
    monkeypatch.setenv("DW_PAIR", "0")  # det0's box0 may otherwise chain with box1
    monkeypatch.setenv("DW_SIB", "1")
    rt = HipGraphRuntime(g, backend, exact_u8_f16=True)
    sib = [L for L in rt.launches() if L["kernel"].endswith("_sib")]
    # only the detect scales' box0 and cls0: other convs whose inputs reuse
    # the same arena bytes at another time are not siblings
    assert len(sib) == 3, [(L["kernel"], L["ops"]) for L in rt.launches()]
    assert all("box0" in L["ops"] and "cls0" in L["ops"] for L in sib), [L["ops"] for L in sib]
    rt.set_input_f32(info["input"], x)
    rt.run()
    got = gpu_outputs(rt, info)
    ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
    for o, gv in zip(info["outputs"], got):
        np.testing.assert_array_equal(gv, ref[o], err_msg=o)
    monkeypatch.setenv("DW_SIB", "0")
    rt0 = HipGraphRuntime(g, backend, exact_u8_f16=True)
    assert not any(L["kernel"].endswith("_sib") for L in rt0.launches())
    rt0.set_input_f32(info["input"], x)
    rt0.run()
    for o, gv, g0 in zip(info["outputs"], got, gpu_outputs(rt0, info)):
        assert gv.tobytes() == g0.tobytes(), o


@pytest.mark.parametrize("size,batch", [(96, 2), (640, 32)])
def test_f16_graph_siblings_same_bytes(backend, monkeypatch, size, batch):
    # The fp16 graph's box0 and cls0 of each detect scale as one GEMM
    # (DW_SIB=1) and as two launches (=0): every output is summed over K in
    # the same k-step order either way, so the same f16 values; within the
    # fp16 tolerance of the oracle at the small size.
    g, info = yolo.f16_graph(batch=batch, size=size)
    x = yolo.input_images(batch, size)
    outs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("DW_SIB", mode)
        rt = HipGraphRuntime(g, backend)
        sib = [L["ops"] for L in rt.launches() if L["kernel"].endswith("_sib")]
        print(f"{size} DW_SIB={mode}: {len(sib)} sibling launches", flush=True)
        assert len(sib) == (3 if mode == "1" else 0), sib
        assert all("box0" in o and "cls0" in o for o in sib), sib
        rt.set_input_f32(info["input"], x)
        rt.run()
        outs[mode] = gpu_outputs(rt, info)
        del rt
    for o, a, b in zip(info["outputs"], outs["0"], outs["1"]):
        np.testing.assert_array_equal(a, b, err_msg=o)
    if size == 96:
        ref = oracle_run(g, {info["input"]: synth.f16_bits(x)})
        for o, gv in zip(info["outputs"], outs["1"]):
            assert rel_err(oracle.f16_to_f32(gv), oracle.f16_to_f32(ref[o])) <= 1e-2, o


def test_int8_benchmark_graph_siblings_same_bytes(backend, monkeypatch):
    # the benchmark's 640 x 640 batch-32 graph with every sibling pair fused
    # and with none: the same bytes on every output
    from dragonwing_edge_rs_amd import workloads

    g, inputs, outs, work, extra = workloads.yolov8n_int8(backend)
    monkeypatch.setenv("DW_PAIR", "0")  # det0's box0 may otherwise chain with box1
    res = []
    for v in ("1", "0"):
        monkeypatch.setenv("DW_SIB", v)
        rt = HipGraphRuntime(g, backend)
        n = sum(L["kernel"].endswith("_sib") for L in rt.launches())
        assert n == (3 if v == "1" else 0), n
        for k, val in inputs.items():
            rt.set_input_bytes(k, val)
        rt.run()
        res.append([rt.get_output_bytes(o).tobytes() for o in outs])
        del rt
    assert res[0] == res[1]


def stem_u8_graph(n, h, w, co, seed):
    """A three-channel 3x3 stride-2 stem kept fp16 (f16 weights) whose
    result is quantized to u8 and run through the SiLU table, as the INT8
    graph's first layer; weights large enough that f16 subnormal inputs
    reach the output bytes."""
    from dragonwing_edge_rs_amd.graph import GRAPH_F32, Graph

    r = np.random.default_rng(seed)
    g = Graph(GRAPH_F32)
    g.add_tensor("x", (n, h, w, 3))
    g.add_initializer("w", r.normal(0, 500.0, (3, 3, 3, co)).astype(np.float32))
    g.add_initializer("b", r.normal(0, 0.5, co).astype(np.float32))
    ho, wo = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    for t in ("s", "sg", "act"):
        g.add_tensor(t, (n, ho, wo, co))
    g.add_op("stem", "Conv", ["x", "w", "b"], ["s"], kernel_shape=(3, 3), strides=(2, 2), pads=(1, 1, 1, 1))
    g.add_op("sig", "Sigmoid", ["s"], ["sg"])
    g.add_op("mul", "Mul", ["s", "sg"], ["act"])
    g.set_io(["x"], ["act"])
    g.set_activation_range("x", -1e-3, 1e-3)
    g.set_activation_range("s", -4.0, 4.0)
    g.set_activation_range("sg", 0.0, 1.0)
    g.set_activation_range("act", -0.3, 4.0)
    g.quantize_qdq(["stem"])
    return g, (n, ho, wo, co)


def stem_u8_inputs(n, h, w, seed):
    """f16 inputs of magnitude <= 1e-3; image 0 entirely f16 subnormals (every
    wave on the reference's half-value decode), the others with one
    subnormal in every eighth row and a block of zeros at the corner."""
    r = np.random.default_rng(seed)
    xb = synth.f16_bits(r.uniform(-1e-3, 1e-3, (n, h, w, 3)).astype(np.float32))
    xb[0] = r.integers(1, 0x400, (h, w, 3)).astype(np.uint16) | (r.integers(0, 2, (h, w, 3)).astype(np.uint16) << 15)
    for i in range(1, n):
        for row in r.choice(h, size=max(1, h // 8), replace=False):
            xb[i, row, r.integers(0, w), r.integers(0, 3)] = np.uint16(r.integers(1, 0x400))
        xb[i, : h // 4, : w // 4] = 0
    return xb


@pytest.mark.parametrize("n,h,w,co", [
    (2, 16, 32, 16),    # one partial workgroup
    (3, 64, 96, 32),    # two 16-channel chunks, many waves
    (2, 18, 36, 16),    # rows of ragged 256-pixel blocks
])
def test_int8_stem_subnormal_inputs_bit_exact(backend, monkeypatch, n, h, w, co):
    # the INT8 graph's fp16 stem with a u8 output (conv, QuantizeLinear, the
    # SiLU table in one launch) on inputs whose f16 subnormals reach the output
    # bytes: the reference's half-value decode, zero blocks and the padded
    # borders give the oracle's bytes, on the padded-window kernel
    # (stem_pad_u8: out-of-image taps as +0, packed inputs widened in the FMA
    # unless the wave holds a subnormal) and on the one-pixel kernel that
    # skips them (DW_STEM_PAD=0)
    g, shp = stem_u8_graph(n, h, w, co, seed=7 + co)
    xb = stem_u8_inputs(n, h, w, seed=8 + h)
    ref = oracle_run(g, {"x": xb})["act"]
    # the test is sensitive to the decode: IEEE-widened subnormals (the
    # reference decode of twice the value) change the output bytes
    sub = ((xb & 0x7C00) == 0) & ((xb & 0x3FF) != 0) & ((xb & 0x3FF) < 0x200)
    x2 = xb.copy()
    x2[sub] = ((xb[sub] & 0x3FF) * 2) | (xb[sub] & 0x8000)
    assert np.mean(oracle_run(g, {"x": x2})["act"] != ref) > 0.01
    for mode, kernel in (("1", "stem_pad_u8"), ("0", "direct_conv")):
        monkeypatch.setenv("DW_STEM_PAD", mode)
        rt = HipGraphRuntime(g, backend)
        assert [L["kernel"] for L in rt.launches()] == [kernel]
        rt.set_input_bytes("x", xb)
        rt.run()
        np.testing.assert_array_equal(rt.get_output_bytes("act").reshape(shp), ref, err_msg=kernel)
    assert len(np.unique(ref)) > 50
