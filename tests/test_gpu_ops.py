"""GPU parity of the op-level C ABI against the oracle (dragonwing-cpu
restatement), on the same seeded inputs.

Bars: bit-exact for every integer path and for the fp32/fp16 kernels that
keep the reference accumulation order; fp16 MFMA convolution within
max|gpu - ref| <= 1e-2 * max|ref|; fp16 paths that call expf (SiLU,
sigmoid) within the same fp16 bar (the GPU expf and glibc expf may differ
in the last bit, which can flip an f16 rounding).
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
import dragonwing_edge_rs_amd as dw
from dragonwing_edge_rs_amd import ops, synth

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def f16v(bits):
    return oracle.f16_to_f32(bits)


# --------------------------------------------------------------------------
# Backend contract (backend.rs:127-199)
# --------------------------------------------------------------------------
def test_backend_roundtrip_and_errors(backend):
    assert backend.name() == "hip-gfx950"
    data = np.arange(1000, dtype=np.uint8)
    buf = backend.from_numpy(data)
    assert buf.len_bytes() == 1000
    out = np.zeros_like(data)
    backend.download(buf, out)
    np.testing.assert_array_equal(out, data)
    with pytest.raises(dw.HipError) as e:
        backend.upload(buf, np.zeros(999, np.uint8))
    assert e.value.code == -4
    with pytest.raises(dw.HipError):
        backend.download(buf, np.zeros(1001, np.uint8))
    empty = backend.alloc(0)
    backend.upload(empty, np.zeros(0, np.uint8))
    backend.synchronize()


# --------------------------------------------------------------------------
# fp32 conv + bias + ReLU (the single-op fp32 workload, 1x64x56x56, 3x3)
# --------------------------------------------------------------------------
def run_conv_f32(be, x, k, b, stride, pad, act):
    n, h, w, ci = x.shape
    kh, kw, _, co = k.shape
    ho, wo = oracle.out_hw(h, w, kh, kw, stride, stride, pad, pad)
    bx, bk = be.from_numpy(x), be.from_numpy(k)
    bb = be.from_numpy(b) if b is not None else None
    by = be.alloc(n * ho * wo * co * 4)
    ops.conv2d_bias_act_f32_nhwc(be, bx, bk, bb, by, n, h, w, ci, co, kh, kw, stride, stride, pad, pad, act)
    return be.to_numpy(by, np.float32, (n, ho, wo, co))


def test_conv_f32_bias_relu_full_workload_bit_exact(backend):
    x, k, b = synth.conv_f32_case(0)
    got = run_conv_f32(backend, x, k, b, 1, 1, ops.ACT_RELU)
    ref = oracle.relu_f32(oracle.bias_add_f32(oracle.conv2d_f32_nhwc(x, k, (1, 1), (1, 1)), b))
    np.testing.assert_array_equal(got, ref)
    assert rel_err(got, ref) <= 1e-3


@pytest.mark.parametrize("shape", [(2, 9, 7, 5, 6, 3, 2, 1), (1, 6, 5, 3, 16, 3, 2, 1),
                                   (3, 5, 5, 4, 12, 1, 1, 0), (1, 1, 1, 8, 8, 3, 1, 1)])
def test_conv_f32_ragged_bit_exact(backend, shape):
    n, h, w, ci, co, k, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.uniform(-1, 1, (n, h, w, ci)).astype(np.float32)
    kk = rng.uniform(-1, 1, (k, k, ci, co)).astype(np.float32)
    got = run_conv_f32(backend, x, kk, None, s, p, ops.ACT_NONE)
    np.testing.assert_array_equal(got, oracle.conv2d_f32_nhwc(x, kk, (s, s), (p, p)))


@pytest.mark.parametrize("shape", [(2, 9, 7, 32, 40, 3, 2, 1), (1, 11, 13, 16, 96, 3, 1, 1),
                                   (3, 6, 5, 48, 33, 5, 1, 2)])
def test_conv_f32_wide_channels_bit_exact(backend, shape):
    # c_in a multiple of 16 (vector input loads), channel counts that are not
    # a multiple of the per-thread channel group, pixel counts that end
    # part-way through a wavefront, 5x5 taps; bias and ReLU.
    n, h, w, ci, co, k, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.uniform(-1, 1, (n, h, w, ci)).astype(np.float32)
    kk = rng.uniform(-1, 1, (k, k, ci, co)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, (co,)).astype(np.float32)
    got = run_conv_f32(backend, x, kk, b, s, p, ops.ACT_RELU)
    ref = oracle.relu_f32(oracle.bias_add_f32(oracle.conv2d_f32_nhwc(x, kk, (s, s), (p, p)), b))
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("shape", [(2, 37, 41, 64, 20, 3, 1, 1), (1, 20, 23, 32, 8, 3, 1, 1),
                                   (2, 5, 7, 64, 4, 3, 1, 1), (1, 30, 18, 16, 8, 5, 2, 2),
                                   (1, 56, 56, 64, 64, 3, 2, 1), (2, 17, 16, 48, 12, 3, 1, 0)])
def test_conv_f32_tiled_bit_exact(backend, shape):
    # the LDS-tiled kernel (c_in 32 or 64, c_out a multiple of 4, 3x3 at
    # stride 1): several 16 x 16 tiles per image with ragged last tiles, an
    # image smaller than one tile, and shapes it does not take (5x5 at
    # stride 2, c_in 48, stride 2 windows); the tap order and the skipped
    # out-of-image taps of the reference
    n, h, w, ci, co, k, s, p = shape
    rng = np.random.default_rng(sum(shape) + 7)
    x = rng.uniform(-1, 1, (n, h, w, ci)).astype(np.float32)
    kk = rng.uniform(-1, 1, (k, k, ci, co)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, (co,)).astype(np.float32)
    got = run_conv_f32(backend, x, kk, b, s, p, ops.ACT_RELU)
    ref = oracle.relu_f32(oracle.bias_add_f32(oracle.conv2d_f32_nhwc(x, kk, (s, s), (p, p)), b))
    np.testing.assert_array_equal(got, ref)


def test_conv_f32_plain_entry(backend):
    x, k, _ = synth.conv_f32_case(0, c_in=16, c_out=8, h=12, w=12)
    n, h, w, ci = x.shape
    bx, bk, by = backend.from_numpy(x), backend.from_numpy(k), backend.alloc(n * h * w * 8 * 4)
    ops.conv2d_f32_nhwc(backend, bx, bk, by, n, h, w, ci, 8, 3, 3, 1, 1, 1, 1)
    np.testing.assert_array_equal(backend.to_numpy(by, np.float32, (n, h, w, 8)),
                                  oracle.conv2d_f32_nhwc(x, k, (1, 1), (1, 1)))
    with pytest.raises(dw.HipError):  # wrong output size is rejected, not truncated
        ops.conv2d_f32_nhwc(backend, bx, bk, backend.alloc(4), n, h, w, ci, 8, 3, 3, 1, 1, 1, 1)


# --------------------------------------------------------------------------
# QLinearConv u8 x s8 -> u8 (INT8 MFMA)
# --------------------------------------------------------------------------
def run_qconv(be, c, stride, pad):
    x, w = c["x"], c["w"]
    n, h, wd, ci = x.shape
    kh, kw, _, co = w.shape
    ho, wo = oracle.out_hw(h, wd, kh, kw, stride, stride, pad, pad)
    bx, bw = be.from_numpy(x), be.from_numpy(w)
    bb = be.from_numpy(np.asarray(c["bias"], np.int32)) if c["bias"] is not None else None
    by = be.alloc(n * ho * wo * co)
    ops.qlinearconv_u8s8(be, bx, bw, bb, by, n, h, wd, ci, co, kh, kw, stride, stride, pad, pad,
                         c["x_scale"], c["x_zp"], c["w_scales"], c["y_scale"], c["y_zp"])
    return be.to_numpy(by, np.uint8, (n, ho, wo, co))


def oracle_qconv(c, stride, pad):
    return oracle.qlinearconv_u8s8(c["x"], c["w"], c["bias"], (stride, stride), (pad, pad), c["x_scale"],
                                   c["x_zp"], c["w_scales"], c["y_scale"], c["y_zp"])


def test_qlinearconv_full_workload_bit_exact(backend):
    # batch 32, 80x80x128 -> 40x40x256, 3x3 stride 2 pad 1
    c = synth.qlinearconv_case(1)
    got = run_qconv(backend, c, 2, 1)
    ref = oracle_qconv(c, 2, 1)
    assert got.shape == (32, 40, 40, 256)
    np.testing.assert_array_equal(got, ref)
    # not trivially saturated: the outputs span the range
    assert 20 < len(np.unique(ref)) and (ref == 0).mean() < 0.5 and (ref == 255).mean() < 0.5


@pytest.mark.parametrize("geom", [(1, 7, 9, 16, 4, 3, 1, 1), (2, 9, 7, 32, 20, 3, 2, 1),
                                  (1, 5, 8, 48, 80, 1, 1, 0), (1, 13, 11, 64, 64, 3, 2, 1),
                                  (2, 6, 6, 128, 144, 3, 1, 1), (1, 20, 20, 256, 256, 1, 1, 0)])
@pytest.mark.parametrize("x_zp", [128, 0, 201])
def test_qlinearconv_shapes_bit_exact(backend, geom, x_zp):
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(100 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((k, k, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=x_zp, y_scale=0.05, y_zp=128)
    np.testing.assert_array_equal(run_qconv(backend, c, s, p), oracle_qconv(c, s, p))


def channel_tile(co):
    for lim, bc in ((96, 128), (80, 96), (64, 80), (48, 64), (32, 48), (16, 32)):
        if co > lim:
            return bc
    return 16


def igemm_tiles(co):
    """Every (channel tile, pixel blocks per wave) the implicit GEMM accepts
    for c_out = co (the shapes the graph runtime's tuner chooses from)."""
    top = channel_tile(co)
    pad = -(-co // top) * top
    return [(bc, pb) for bc in (128, 96, 80, 64, 48, 32, 16) if bc <= top and pad % bc == 0
            for pb in (4, 2, 1)]


def igemm_sk_tiles(co, ksteps):
    """The persistent small-K tiles (channel tile, pixel blocks, pixel tiles
    per workgroup) for c_out = co and a K of `ksteps` 64-byte k-steps; one
    and three tiles per workgroup (a range that ends part-way is covered)."""
    if not 1 <= ksteps <= 4:
        return []
    top = channel_tile(co)
    pad = -(-co // top) * top
    return [(bc, pb, t) for bc in (128, 64, 32, 16) if bc <= top and pad % bc == 0
            for pb in (4, 2) for t in (1, 3)]


@pytest.mark.parametrize("case", ["ties", "saturation"])
@pytest.mark.parametrize("tile", ["32,4", "32,4,2"])
def test_qlinearconv_requant_ties_and_saturation(backend, case, tile, monkeypatch):
    # The fast epilogues round acc * M by adding 1.5 * 2^23.  "ties": M = 0.5
    # exactly, so every odd accumulator is a tie (round half to even);
    # "saturation": M about 2000, so |acc * M| runs far past 2^22 both ways.
    monkeypatch.setenv("DW_IGEMM_TILE", tile)
    r = synth.Rng(synth.seed_for(800 if case == "ties" else 801))
    n, h, w, ci, co = 2, 9, 10, 32, 32
    if case == "ties":
        x = r.integers((n, h, w, ci), 118, 138).astype(np.uint8)
        wt = r.integers((1, 1, ci, co), -3, 3).astype(np.int8)
        c = dict(x=x, w=wt, bias=r.integers((co,), -40, 40).astype(np.int32),
                 w_scales=np.full(co, 0.5, np.float32), x_scale=1.0, x_zp=128, y_scale=1.0, y_zp=128)
    else:
        x = r.integers((n, h, w, ci), 0, 255).astype(np.uint8)
        wt = r.integers((1, 1, ci, co), -127, 127).astype(np.int8)
        c = dict(x=x, w=wt, bias=r.integers((co,), -4096, 4096).astype(np.int32),
                 w_scales=np.full(co, 0.25, np.float32), x_scale=0.5, x_zp=100, y_scale=6.25e-5, y_zp=3)
    ref = oracle_qconv(c, 1, 0)
    got = run_qconv(backend, c, 1, 0)
    np.testing.assert_array_equal(got, ref)
    if case == "ties":
        assert 10 < len(np.unique(ref)) and (ref == 0).mean() < 0.2 and (ref == 255).mean() < 0.2
    else:
        assert (ref == 0).mean() > 0.2 and (ref == 255).mean() > 0.2


@pytest.mark.parametrize("geom", [(2, 10, 10, 48, 96, 1, 1, 0), (1, 23, 17, 256, 128, 1, 1, 0),
                                  (2, 19, 21, 16, 16, 3, 1, 1), (1, 33, 31, 16, 32, 3, 2, 1),
                                  (3, 9, 13, 128, 20, 1, 1, 0)])
def test_qlinearconv_persistent_tiles_bit_exact(backend, geom, monkeypatch):
    # K of 1 to 4 k-steps: the persistent kernel over every tile it has.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(700 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((k, k, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=131, y_scale=0.05, y_zp=120)
    ref = oracle_qconv(c, s, p)
    tiles = igemm_sk_tiles(co, -(-k * k * ci // 64))
    assert tiles
    for bc, pb, t in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{pb},{t}")
        np.testing.assert_array_equal(run_qconv(backend, c, s, p), ref, err_msg=f"tile {bc},{pb},{t}")


@pytest.mark.parametrize("geom", [(2, 9, 11, 64, 256, 3, 2, 1), (1, 13, 7, 128, 80, 3, 1, 1),
                                  (2, 10, 10, 48, 96, 1, 1, 0), (1, 6, 6, 256, 128, 3, 1, 1)])
def test_qlinearconv_every_tile_bit_exact(backend, geom, monkeypatch):
    # The last case has 36 k-steps, staged through LDS in several chunks.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(500 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((k, k, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=128, y_scale=0.05, y_zp=128)
    ref = oracle_qconv(c, s, p)
    for bc, pb in igemm_tiles(co):
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{pb}")
        np.testing.assert_array_equal(run_qconv(backend, c, s, p), ref, err_msg=f"tile {bc},{pb}")


@pytest.mark.parametrize("geom", [(2, 9, 11, 64, 256, 3, 2, 1), (1, 13, 7, 128, 80, 3, 1, 1),
                                  (2, 10, 10, 48, 96, 1, 1, 0), (1, 6, 6, 256, 128, 3, 1, 1),
                                  (2, 5, 7, 272, 48, 3, 1, 1)])
def test_qlinearconv_streamed_tiles_bit_exact(backend, geom, monkeypatch):
    # The streamed-weight kernel over every tile: K of 2 to 37 k-steps, so
    # the weight ring wraps several times and ends part-way through it.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(900 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((k, k, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=126, y_scale=0.05, y_zp=133)
    ref = oracle_qconv(c, s, p)
    for bc, pb in igemm_tiles(co):
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{pb},-1")
        np.testing.assert_array_equal(run_qconv(backend, c, s, p), ref, err_msg=f"tile {bc},{pb},-1")


@pytest.mark.parametrize("geom", [(2, 8, 80, 64, 64, 3, 1, 1), (1, 4, 160, 16, 32, 3, 1, 1),
                                  (2, 16, 40, 128, 96, 3, 1, 1), (1, 8, 80, 80, 80, 3, 1, 1),
                                  (1, 2, 160, 48, 16, 3, 1, 1)])
def test_qlinearconv_row_tiles_bit_exact(backend, geom, monkeypatch):
    # The row-tile kernel (3x3, stride 1, whole rows of 320 pixels staged in
    # LDS with their halo) over every channel tile it has; zero points other
    # than 128 make the padding pattern matter.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(950 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((k, k, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=119, y_scale=0.05, y_zp=140)
    ref = oracle_qconv(c, s, p)
    tiles = [bc for bc, pb in igemm_tiles(co) if pb == 4 and bc <= 96]
    assert tiles
    for bc in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},4,-2")
        np.testing.assert_array_equal(run_qconv(backend, c, s, p), ref, err_msg=f"tile {bc},4,-2")


def band_tiles(h, w, ci, co, esize=1, waves=8, stride=1):
    """The band-tile kernel's (channel tile, band height, tile code) triples
    for a 3x3 padding-1 conv of stride 1 or 2 on an h x w map with `waves`
    waves (8: code -4, 16: code -5): channel tiles of 128, 80, 64, 32 or 16
    that divide the padded c_out (16 waves: at most 64 unless the epilogue
    is the plain u8 requantize), heights that divide the output height with
    at least one 16-pixel block per wave, the input tile (s (rows - 1) + 3
    rows of s (wo - 1) + 3 pixels) within the start-up loads (8192 units)
    and everything within the 160 KB of LDS."""
    top = channel_tile(co)
    pad = -(-co // top) * top
    cu = ci * esize // 16
    ks = -(-9 * ci * esize // 64)
    ho, wo = (h - 1) // stride + 1, (w - 1) // stride + 1
    tw = stride * (wo - 1) + 3
    out = []
    for bc in (128, 80, 64, 32, 16):
        if pad % bc or (waves == 16 and bc > 64 and esize != 1):
            continue
        for rows in range(1, ho + 1):
            tr = stride * (rows - 1) + 3
            if ho % rows or rows * wo < 16 * waves or tr * tw * cu > 16 * 512:
                continue
            w_off = -(-(256 + 8 * bc + ks * 16) // 16) * 16
            lds = w_off + ks * bc * 64 + tr * tw * (cu | 1) * 16 + waves * 16 * (bc + 16 if bc % 32 == 0 else bc)
            if lds <= 160 * 1024:
                out.append((bc, rows, -4 if waves == 8 else -5))
    return out


@pytest.mark.parametrize("geom,x_zp", [((2, 10, 20, 64, 80), 119), ((1, 24, 16, 32, 32), 128),
                                       ((3, 6, 40, 128, 128), 7), ((1, 14, 22, 16, 16), 140),
                                       ((2, 9, 30, 64, 256), 100)])
def test_qlinearconv_band_tiles_bit_exact(backend, geom, x_zp, monkeypatch):
    # The band-tile kernel (3x3 stride 1: R whole rows staged in LDS, 8
    # waves walking contiguous ranges of 16-pixel blocks, the last chunk of
    # a range part-full) over every channel tile and band height it accepts;
    # bands whose pixel count is not a multiple of 16 and of 8 blocks, and
    # zero points other than 128 (the padding pattern).
    n, h, w, ci, co = geom
    r = synth.Rng(synth.seed_for(1300 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((3, 3, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=x_zp, y_scale=0.05, y_zp=133)
    ref = oracle_qconv(c, 1, 1)
    tiles = band_tiles(h, w, ci, co) + band_tiles(h, w, ci, co, waves=16)
    assert tiles
    for bc, rows, code in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{rows},{code}")
        np.testing.assert_array_equal(run_qconv(backend, c, 1, 1), ref, err_msg=f"tile {bc},{rows},{code}")


@pytest.mark.parametrize("geom,x_zp", [((2, 24, 64, 64, 128), 119), ((1, 31, 63, 32, 64), 128),
                                       ((1, 36, 48, 64, 80), 7), ((2, 18, 30, 128, 64), 140)])
def test_qlinearconv_band_tiles_stride2_bit_exact(backend, geom, x_zp, monkeypatch):
    # The band-tile kernel at stride 2 (2 R + 1 input rows per band, each
    # row's even columns stored before its odd ones): every channel tile and
    # band height it accepts, odd input sizes (the last output row and
    # column read one padding row and column), zero points other than 128.
    n, h, w, ci, co = geom
    r = synth.Rng(synth.seed_for(1700 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((3, 3, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=x_zp, y_scale=0.05, y_zp=133)
    ref = oracle_qconv(c, 2, 1)
    tiles = band_tiles(h, w, ci, co, stride=2) + band_tiles(h, w, ci, co, waves=16, stride=2)
    assert tiles
    print(f"{geom}: {len(tiles)} band tiles", flush=True)
    for bc, rows, code in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{rows},{code}")
        np.testing.assert_array_equal(run_qconv(backend, c, 2, 1), ref, err_msg=f"tile {bc},{rows},{code}")


def wide_tiles(co):
    """The wide-tile kernel's channel tiles for c_out = co (input rows of
    whole 128-byte units)."""
    top = channel_tile(co)
    pad = -(-co // top) * top
    return [bc for bc in (256, 128, 64) if pad % bc == 0 and not (bc > 64 and co <= bc // 2)]


@pytest.mark.parametrize("geom,x_zp", [((2, 9, 11, 128, 256, 3, 2, 1), 128), ((1, 13, 7, 256, 128, 3, 1, 1), 119),
                                       ((2, 10, 10, 128, 64, 1, 1, 0), 140), ((1, 6, 6, 384, 256, 1, 1, 0), 128),
                                       ((2, 20, 20, 128, 128, 3, 2, 1), 100), ((3, 5, 3, 128, 192, 3, 1, 1), 7)])
def test_qlinearconv_wide_tiles_bit_exact(backend, geom, x_zp, monkeypatch):
    # The wide-tile kernel (k-step pairs staged through LDS with swizzled
    # whole-line loads, 256-pixel workgroups) over every channel tile it has;
    # ragged pixel counts, padding with zero points other than 128, 1x1 and
    # strided 3x3 layers.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(1100 + sum(geom)))
    c = dict(x=r.integers((n, h, w, ci), 0, 255).astype(np.uint8),
             w=r.integers((k, k, ci, co), -127, 127).astype(np.int8),
             bias=r.integers((co,), -4096, 4096).astype(np.int32),
             w_scales=r.log_uniform((co,), 1e-3, 1e-2), x_scale=0.02, x_zp=x_zp, y_scale=0.05, y_zp=131)
    ref = oracle_qconv(c, s, p)
    tiles = wide_tiles(co)
    assert tiles
    for bc in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},4,-3")
        np.testing.assert_array_equal(run_qconv(backend, c, s, p), ref, err_msg=f"tile {bc},4,-3")


def test_qlinearconv_full_workload_wide_bit_exact(backend, monkeypatch):
    # batch 32, 80x80x128 -> 40x40x256 on the wide-tile kernel, every tile
    c = synth.qlinearconv_case(1)
    ref = oracle_qconv(c, 2, 1)
    for bc in (256, 128, 64):
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},4,-3")
        np.testing.assert_array_equal(run_qconv(backend, c, 2, 1), ref, err_msg=f"tile {bc},4,-3")


def test_qlinearconv_golden_fixtures(backend):
    cases = json.loads((GOLDEN / "qlinear_cases.json").read_text())["qlinearconv"]
    for g in cases:
        c = dict(x=np.array(g["x"], np.uint8).reshape(g["x_shape"]),
                 w=np.array(g["w"], np.int8).reshape(g["w_shape"]), bias=np.array(g["bias"], np.int32),
                 w_scales=np.array(g["w_scales"], np.float32), x_scale=g["x_scale"], x_zp=g["x_zp"],
                 y_scale=g["y_scale"], y_zp=g["y_zp"])
        got = run_qconv(backend, c, g["stride"][0], g["pad"][0])
        np.testing.assert_array_equal(got.ravel(), g["y"], err_msg=g["name"])


def test_qlinearconv_rejects_unsupported(backend):
    x = backend.alloc(1 * 4 * 4 * 8)
    w = backend.alloc(9 * 8 * 4)
    y = backend.alloc(1 * 4 * 4 * 4)
    with pytest.raises(dw.HipError) as e:  # c_in = 8 is not a multiple of 16
        ops.qlinearconv_u8s8(backend, x, w, None, y, 1, 4, 4, 8, 4, 3, 3, 1, 1, 1, 1, 0.02, 128,
                             np.ones(4, np.float32), 0.05, 128)
    assert e.value.code == -2


# --------------------------------------------------------------------------
# Reference INT8 ops (symmetric s8)
# --------------------------------------------------------------------------
def test_conv2d_i8_and_requant_relu_bit_exact(backend):
    r = synth.Rng(synth.seed_for(7))
    n, h, w, ci, co = 2, 11, 9, 32, 24
    x = r.integers((n, h, w, ci), -128, 127).astype(np.int8)
    k = r.integers((3, 3, ci, co), -127, 127).astype(np.int8)
    bx, bk = backend.from_numpy(x), backend.from_numpy(k)
    for s in (1, 2):
        ho, wo = oracle.out_hw(h, w, 3, 3, s, s, 1, 1)
        acc_ref = oracle.conv2d_i8_nhwc(x, k, (s, s), (1, 1))
        by = backend.alloc(n * ho * wo * co * 4)
        ops.conv2d_i8_nhwc(backend, bx, bk, by, n, h, w, ci, co, 3, 3, s, s, 1, 1)
        np.testing.assert_array_equal(backend.to_numpy(by, np.int32, acc_ref.shape), acc_ref)
        for relu in (0, 1):
            scale = 0.0023
            ref = oracle.requantize_i32_to_i8(acc_ref, scale)
            if relu:
                ref = oracle.relu_i8(ref)
            bq = backend.alloc(n * ho * wo * co)
            ops.conv2d_requant_relu_i8(backend, bx, bk, bq, n, h, w, ci, co, 3, 3, s, s, 1, 1, scale, relu)
            np.testing.assert_array_equal(backend.to_numpy(bq, np.int8, ref.shape), ref)


def test_int8_elementwise_bit_exact(backend):
    r = synth.Rng(synth.seed_for(8))
    acc = r.integers((4099,), -40000, 40000).astype(np.int32)
    a = r.integers((4099,), -128, 127).astype(np.int8)
    b = r.integers((4099,), -128, 127).astype(np.int8)
    f = r.uniform((4099,), -20.0, 20.0)
    n = 4099
    bacc, ba, bb, bf = map(backend.from_numpy, (acc, a, b, f))
    y8 = backend.alloc(n)
    ops.requantize_i32_to_i8(backend, bacc, y8, n, 0.0031)
    np.testing.assert_array_equal(backend.to_numpy(y8, np.int8, n), oracle.requantize_i32_to_i8(acc, 0.0031))
    ops.add_i8(backend, ba, bb, y8, n, 0.7, 0.45)
    np.testing.assert_array_equal(backend.to_numpy(y8, np.int8, n), oracle.add_i8(a, b, 0.7, 0.45))
    ops.relu_i8(backend, ba, y8, n)
    np.testing.assert_array_equal(backend.to_numpy(y8, np.int8, n), oracle.relu_i8(a))
    ops.quantize_f32_to_i8(backend, bf, y8, n, 0.13)
    np.testing.assert_array_equal(backend.to_numpy(y8, np.int8, n), oracle.quantize_f32_to_i8(f, 0.13))
    yf = backend.alloc(n * 4)
    ops.dequantize_i8_to_f32(backend, ba, yf, n, 0.07)
    np.testing.assert_array_equal(backend.to_numpy(yf, np.float32, n), oracle.dequantize_i8_to_f32(a, 0.07))


def test_onnx_quant_elementwise_bit_exact(backend):
    r = synth.Rng(synth.seed_for(9))
    n = 5000
    xa = r.integers((n,), 0, 255).astype(np.uint8)
    xb = r.integers((n,), 0, 255).astype(np.uint8)
    xh = synth.f16_bits(r.normal((n,), 0.0, 3.0))
    ba, bb, bh = map(backend.from_numpy, (xa, xb, xh))
    y = backend.alloc(n)
    ops.qlinear_add_u8(backend, ba, bb, y, n, 0.031, 120, 0.017, 131, 0.04, 125)
    np.testing.assert_array_equal(backend.to_numpy(y, np.uint8, n),
                                  oracle.qlinear_add_u8(xa, xb, 0.031, 120, 0.017, 131, 0.04, 125))
    ops.quantize_linear_f16_u8(backend, bh, y, n, 0.037, 128)
    np.testing.assert_array_equal(backend.to_numpy(y, np.uint8, n), oracle.quantize_linear_f16_u8(xh, 0.037, 128))
    yh = backend.alloc(n * 2)
    ops.dequantize_linear_u8_f16(backend, ba, yh, n, 0.021, 128)
    np.testing.assert_array_equal(backend.to_numpy(yh, np.uint16, n),
                                  oracle.dequantize_linear_u8_f16(xa, 0.021, 128))
    lut = oracle.silu_lut_u8(0.05, 128, 0.03, 128)
    ops.lut_u8(backend, ba, y, n, lut)
    np.testing.assert_array_equal(backend.to_numpy(y, np.uint8, n), lut[xa])


# --------------------------------------------------------------------------
# fp16 convolutions
# --------------------------------------------------------------------------
def run_conv_f16(be, xh, kh_, bh, stride, pad, act, exact):
    n, h, w, ci = xh.shape
    kh, kw, _, co = kh_.shape
    ho, wo = oracle.out_hw(h, w, kh, kw, stride, stride, pad, pad)
    bx, bk = be.from_numpy(xh), be.from_numpy(kh_)
    bb = be.from_numpy(bh) if bh is not None else None
    by = be.alloc(n * ho * wo * co * 2)
    ops.conv2d_bias_act_f16_nhwc(be, bx, bk, bb, by, n, h, w, ci, co, kh, kw, stride, stride, pad, pad,
                                 act, exact)
    return be.to_numpy(by, np.uint16, (n, ho, wo, co))


def oracle_conv_f16(xh, kh_, bh, stride, pad, act):
    y = oracle.conv2d_fp16_nhwc(xh, kh_, (stride, stride), (pad, pad))
    if bh is not None:
        y = oracle.bias_add_f16(y, bh)
    if act == ops.ACT_RELU:
        y = oracle.relu_fp16(y)
    elif act == ops.ACT_SILU:
        y = oracle.silu_fp16(y)
    return y


@pytest.mark.parametrize("geom", [(2, 16, 16, 16, 32, 3, 2, 1), (1, 20, 20, 64, 64, 3, 1, 1),
                                  (2, 10, 10, 80, 80, 3, 1, 1), (1, 12, 12, 128, 256, 1, 1, 0),
                                  (1, 9, 7, 48, 16, 3, 1, 1), (1, 17, 9, 32, 144, 3, 2, 1)])
@pytest.mark.parametrize("act", [ops.ACT_NONE, ops.ACT_SILU])
def test_conv_f16_mfma_within_tolerance(backend, geom, act):
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(200 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, (1.0 / (k * k * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    got = run_conv_f16(backend, xh, kh_, bh, s, p, act, exact=False)
    ref = oracle_conv_f16(xh, kh_, bh, s, p, act)
    assert rel_err(f16v(got), f16v(ref)) <= 1e-2


def test_conv_f16_mfma_every_tile_identical(backend, monkeypatch):
    # Tile shapes split the work differently but accumulate every output
    # over the same k-steps in the same order: results agree bit for bit.
    n, h, w, ci, co, k, s, p = 2, 11, 9, 64, 128, 3, 1, 1
    r = synth.Rng(synth.seed_for(600))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, (1.0 / (k * k * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, s, p, ops.ACT_SILU)
    first = None
    for bc, pb in igemm_tiles(co):
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{pb}")
        got = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
        assert rel_err(f16v(got), f16v(ref)) <= 1e-2
        if first is None:
            first = got
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},{pb}")


def test_conv_f16_persistent_tiles_identical(backend, monkeypatch):
    # 1x1 over 64 f16 channels: two k-steps, so the persistent kernel applies;
    # it sums the same k-steps in the same order as the other tiles.
    n, h, w, ci, co, k, s, p = 2, 13, 11, 64, 64, 1, 1, 0
    r = synth.Rng(synth.seed_for(601))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, (1.0 / (k * k * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, s, p, ops.ACT_SILU)
    monkeypatch.setenv("DW_IGEMM_TILE", "64,4")
    first = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
    assert rel_err(f16v(first), f16v(ref)) <= 1e-2
    for bc, pb, t in igemm_sk_tiles(co, 2):
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{pb},{t}")
        got = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},{pb},{t}")


def test_conv_f16_streamed_tiles_identical(backend, monkeypatch):
    # 3x3 over 64 f16 channels: 18 k-steps.  The streamed-weight kernel sums
    # the same k-steps in the same order as the staged one.
    n, h, w, ci, co, k, s, p = 2, 11, 9, 64, 96, 3, 1, 1
    r = synth.Rng(synth.seed_for(602))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, (1.0 / (k * k * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, s, p, ops.ACT_SILU)
    monkeypatch.setenv("DW_IGEMM_TILE", "32,4")
    first = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
    assert rel_err(f16v(first), f16v(ref)) <= 1e-2
    for bc, pb in igemm_tiles(co):
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{pb},-1")
        got = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},{pb},-1")


@pytest.mark.parametrize("geom", [(2, 16, 40, 64, 64), (1, 8, 80, 32, 48), (1, 4, 160, 16, 32)])
def test_conv_f16_row_tiles_identical(backend, monkeypatch, geom):
    # 3x3 stride 1 over whole rows of 40, 80 and 160 pixels: the row-tile
    # kernel stages the input rows in LDS and sums the same k-steps in the
    # same order as the staged kernel, so the results are identical.
    n, h, w, ci, co = geom
    r = synth.Rng(synth.seed_for(603 + w))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((3, 3, ci, co), 0.0, (1.0 / (9 * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, 1, 1, ops.ACT_SILU)
    monkeypatch.setenv("DW_IGEMM_TILE", "16,4")
    first = run_conv_f16(backend, xh, kh_, bh, 1, 1, ops.ACT_SILU, exact=False)
    assert rel_err(f16v(first), f16v(ref)) <= 1e-2
    for bc in (16, 32, 48, 64):
        if co % bc:
            continue
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},4,-2")
        got = run_conv_f16(backend, xh, kh_, bh, 1, 1, ops.ACT_SILU, exact=False)
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},4,-2")


@pytest.mark.parametrize("geom", [(2, 16, 16, 32, 32), (1, 10, 40, 64, 80), (2, 8, 18, 128, 64)])
def test_conv_f16_band_tiles_identical(backend, monkeypatch, geom):
    # The band-tile kernel in fp16: the same k-steps summed in the same order
    # as the staged kernel, so the results are identical.
    n, h, w, ci, co = geom
    r = synth.Rng(synth.seed_for(1400 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((3, 3, ci, co), 0.0, (1.0 / (9 * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, 1, 1, ops.ACT_SILU)
    monkeypatch.setenv("DW_IGEMM_TILE", "16,4")
    first = run_conv_f16(backend, xh, kh_, bh, 1, 1, ops.ACT_SILU, exact=False)
    assert rel_err(f16v(first), f16v(ref)) <= 1e-2
    tiles = band_tiles(h, w, ci, co, esize=2) + band_tiles(h, w, ci, co, esize=2, waves=16)
    assert tiles
    for bc, rows, code in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{rows},{code}")
        got = run_conv_f16(backend, xh, kh_, bh, 1, 1, ops.ACT_SILU, exact=False)
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},{rows},{code}")


@pytest.mark.parametrize("geom", [(2, 20, 40, 32, 64), (1, 31, 47, 16, 32)])
def test_conv_f16_band_tiles_stride2_identical(backend, monkeypatch, geom):
    # The fp16 band-tile kernel at stride 2 sums the staged kernel's k-steps
    # in its order: identical results, odd input sizes included.
    n, h, w, ci, co = geom
    r = synth.Rng(synth.seed_for(1800 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((3, 3, ci, co), 0.0, (1.0 / (9 * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, 2, 1, ops.ACT_SILU)
    monkeypatch.setenv("DW_IGEMM_TILE", "16,4")
    first = run_conv_f16(backend, xh, kh_, bh, 2, 1, ops.ACT_SILU, exact=False)
    assert rel_err(f16v(first), f16v(ref)) <= 1e-2
    tiles = band_tiles(h, w, ci, co, esize=2, stride=2) + band_tiles(h, w, ci, co, esize=2, waves=16, stride=2)
    assert tiles
    for bc, rows, code in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},{rows},{code}")
        got = run_conv_f16(backend, xh, kh_, bh, 2, 1, ops.ACT_SILU, exact=False)
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},{rows},{code}")


@pytest.mark.parametrize("geom", [(2, 11, 9, 64, 128, 3, 1, 1), (2, 20, 18, 128, 64, 3, 2, 1),
                                  (1, 12, 10, 64, 256, 1, 1, 0), (3, 7, 5, 192, 192, 3, 1, 1)])
def test_conv_f16_wide_tiles_identical(backend, monkeypatch, geom):
    # Input rows of whole 128-byte units (c_in % 64 == 0): the wide-tile
    # kernel stages k-step pairs through LDS and sums the same k-steps in the
    # same order as the staged kernel, so the results are identical.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(640 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, (1.0 / (k * k * ci)) ** 0.5))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    ref = oracle_conv_f16(xh, kh_, bh, s, p, ops.ACT_SILU)
    monkeypatch.setenv("DW_IGEMM_TILE", "16,4")
    first = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
    assert rel_err(f16v(first), f16v(ref)) <= 1e-2
    tiles = wide_tiles(co)
    assert tiles
    for bc in tiles:
        monkeypatch.setenv("DW_IGEMM_TILE", f"{bc},4,-3")
        got = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_SILU, exact=False)
        np.testing.assert_array_equal(got, first, err_msg=f"tile {bc},4,-3")


@pytest.mark.parametrize("geom", [(2, 32, 32, 3, 16, 3, 2, 1), (1, 12, 12, 64, 64, 1, 1, 0),
                                  (1, 10, 10, 80, 80, 1, 1, 0), (1, 17, 15, 3, 16, 3, 2, 1),
                                  (2, 20, 22, 3, 16, 3, 2, 0), (1, 9, 12, 3, 32, 3, 2, 1),
                                  (1, 11, 10, 3, 16, 3, 1, 1)])
def test_conv_f16_exact_order_bit_exact(backend, geom):
    # The 3-channel stem shapes take the row-load path (even width and
    # column stride, either pad parity) or the per-value loads (odd width,
    # stride 1); subnormal inputs are planted for the reference's decode.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(300 + sum(geom)))
    xh = synth.f16_bits(r.uniform((n, h, w, ci), 0.0, 1.0))
    xh.ravel()[::97] = np.uint16(0x0005)
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, 0.2))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    got = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_NONE, exact=True)
    np.testing.assert_array_equal(got, oracle_conv_f16(xh, kh_, bh, s, p, ops.ACT_NONE))
    got = run_conv_f16(backend, xh, kh_, bh, s, p, ops.ACT_RELU, exact=True)
    np.testing.assert_array_equal(got, oracle_conv_f16(xh, kh_, bh, s, p, ops.ACT_RELU))


@pytest.mark.parametrize("geom", [(1, 9, 7, 16, 80, 1, 1, 0), (2, 33, 31, 64, 64, 1, 1, 0),
                                  (1, 40, 40, 80, 80, 1, 1, 0), (3, 11, 13, 32, 40, 1, 2, 0),
                                  (1, 5, 5, 8, 4, 1, 1, 0), (8, 20, 20, 64, 20, 1, 1, 0)])
def test_conv_f16_exact_1x1_bit_exact(backend, geom):
    # The 1x1 exact-order kernel: ragged pixel counts, stride 2, and c_out
    # values that select every channels-per-wave / pixels-per-lane shape.
    n, h, w, ci, co, k, s, p = geom
    r = synth.Rng(synth.seed_for(700 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, ci), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((k, k, ci, co), 0.0, 0.2))
    bh = synth.f16_bits(r.normal((co,), 0.0, 0.1))
    # (ReLU, not SiLU: bit-exact SiLU would need the host libm's expf)
    for act in (ops.ACT_NONE, ops.ACT_RELU):
        got = run_conv_f16(backend, xh, kh_, bh, s, p, act, exact=True)
        np.testing.assert_array_equal(got, oracle_conv_f16(xh, kh_, bh, s, p, act), err_msg=f"act {act}")


def test_conv_f16_subnormal_inputs_follow_reference_decode(backend):
    # dragonwing-cpu widens f16 subnormals at half their IEEE value; the
    # exact-order kernel reproduces it bit for bit.
    xh = np.full((1, 4, 4, 8), 0x0200, np.uint16)  # subnormal
    kh_ = np.full((1, 1, 8, 8), 0x3C00, np.uint16)  # 1.0
    got = run_conv_f16(backend, xh, kh_, None, 1, 0, ops.ACT_NONE, exact=True)
    np.testing.assert_array_equal(got, oracle_conv_f16(xh, kh_, None, 1, 0, ops.ACT_NONE))


# --------------------------------------------------------------------------
# Depthwise 3x3 fp16 + bias + SiLU (batch 32, 40x40x384)
# --------------------------------------------------------------------------
def test_depthwise_f16_full_workload(backend):
    x, wt, b = synth.dwconv_case(2)
    n, h, w, c = x.shape
    bx, bw, bb = backend.from_numpy(x), backend.from_numpy(wt), backend.from_numpy(b)
    by = backend.alloc(x.nbytes)
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bw, bb, by, n, h, w, c, 3, 3, 1, 1, 1, 1, ops.ACT_SILU)
    got = backend.to_numpy(by, np.uint16, x.shape)
    ref = oracle.silu_fp16(oracle.bias_add_f16(oracle.depthwise_fp16(x, wt, (1, 1), (1, 1)), b))
    assert rel_err(f16v(got), f16v(ref)) <= 1e-2
    # Everything before the expf-based activation is bit-exact:
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bw, bb, by, n, h, w, c, 3, 3, 1, 1, 1, 1, ops.ACT_NONE)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, x.shape),
                                  oracle.bias_add_f16(oracle.depthwise_fp16(x, wt, (1, 1), (1, 1)), b))
    assert np.mean(got != ref) < 1e-3  # f16 flips from expf last-bit differences are rare


@pytest.mark.parametrize("geom", [(1, 5, 11, 12, 1), (2, 13, 10, 4, 2), (1, 9, 17, 20, 1), (3, 8, 19, 36, 2)])
def test_depthwise_f16_sliding_window_shapes(backend, geom):
    # Row lengths that end part-way through a thread's 4 outputs, channel
    # counts that are multiples of 4 but not 8, both strides; bias and no bias.
    n, h, w, c, s = geom
    r = synth.Rng(synth.seed_for(420 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, c), 0.0, 1.0))
    kh_ = synth.f16_bits(r.normal((3, 3, c), 0.0, 0.3))
    bh = synth.f16_bits(r.normal((c,), 0.0, 0.1))
    ho, wo = oracle.out_hw(h, w, 3, 3, s, s, 1, 1)
    bx, bk, bb = backend.from_numpy(xh), backend.from_numpy(kh_), backend.from_numpy(bh)
    by = backend.alloc(n * ho * wo * c * 2)
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bk, bb, by, n, h, w, c, 3, 3, s, s, 1, 1, ops.ACT_NONE)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, (n, ho, wo, c)),
                                  oracle.bias_add_f16(oracle.depthwise_fp16(xh, kh_, (s, s), (1, 1)), bh))
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bk, None, by, n, h, w, c, 3, 3, s, s, 1, 1, ops.ACT_SILU)
    got = backend.to_numpy(by, np.uint16, (n, ho, wo, c))
    ref = oracle.silu_fp16(oracle.depthwise_fp16(xh, kh_, (s, s), (1, 1)))
    assert rel_err(f16v(got), f16v(ref)) <= 1e-2


@pytest.mark.parametrize("geom", [(2, 7, 83, 64, 0), (1, 9, 40, 128, 1), (3, 5, 6, 8, 1), (1, 11, 45, 24, 0),
                                  (1, 1, 1, 64, 0), (2, 4, 41, 72, 1)])
def test_depthwise_f16_stride1_shapes(backend, geom):
    # Stride-1 shapes: wide rows, odd heights, 64- and 8-channel multiples, a
    # 1x1 map; subnormal inputs planted in some (the reference decodes them
    # at half value).
    n, h, w, c, plant = geom
    r = synth.Rng(synth.seed_for(460 + sum(geom)))
    xh = synth.f16_bits(r.normal((n, h, w, c), 0.0, 1.0))
    if plant:
        xh.ravel()[::331] = np.uint16(0x8007)
    kh_ = synth.f16_bits(r.normal((3, 3, c), 0.0, 0.3))
    bh = synth.f16_bits(r.normal((c,), 0.0, 0.1))
    bx, bk, bb = backend.from_numpy(xh), backend.from_numpy(kh_), backend.from_numpy(bh)
    by = backend.alloc(xh.nbytes)
    conv = oracle.depthwise_fp16(xh, kh_, (1, 1), (1, 1))
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bk, bb, by, n, h, w, c, 3, 3, 1, 1, 1, 1, ops.ACT_NONE)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, xh.shape), oracle.bias_add_f16(conv, bh))
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bk, None, by, n, h, w, c, 3, 3, 1, 1, 1, 1, ops.ACT_RELU)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, xh.shape), oracle.relu_fp16(conv))
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bk, bb, by, n, h, w, c, 3, 3, 1, 1, 1, 1, ops.ACT_SILU)
    got = backend.to_numpy(by, np.uint16, xh.shape)
    ref = oracle.silu_fp16(oracle.bias_add_f16(conv, bh))
    assert rel_err(f16v(got), f16v(ref)) <= 1e-2


@pytest.mark.parametrize("geom", [(1, 7, 5, 8, 2), (2, 9, 9, 16, 1), (1, 6, 6, 24, 2)])
def test_depthwise_f32_and_f16_ragged(backend, geom):
    n, h, w, c, s = geom
    r = synth.Rng(synth.seed_for(400 + sum(geom)))
    x = r.normal((n, h, w, c), 0.0, 1.0)
    k = r.normal((3, 3, c), 0.0, 0.3)
    ho, wo = oracle.out_hw(h, w, 3, 3, s, s, 1, 1)
    bx, bk = backend.from_numpy(x), backend.from_numpy(k)
    by = backend.alloc(n * ho * wo * c * 4)
    ops.depthwise_conv2d_f32_nhwc(backend, bx, bk, None, by, n, h, w, c, 3, 3, s, s, 1, 1, ops.ACT_RELU)
    np.testing.assert_array_equal(backend.to_numpy(by, np.float32, (n, ho, wo, c)),
                                  oracle.relu_f32(oracle.depthwise_f32(x, k, (s, s), (1, 1))))
    xh, kh_ = synth.f16_bits(x), synth.f16_bits(k)
    bx, bk = backend.from_numpy(xh), backend.from_numpy(kh_)
    by = backend.alloc(n * ho * wo * c * 2)
    ops.depthwise_conv2d_f16_nhwc(backend, bx, bk, None, by, n, h, w, c, 3, 3, s, s, 1, 1, ops.ACT_NONE)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, (n, ho, wo, c)),
                                  oracle.depthwise_fp16(xh, kh_, (s, s), (1, 1)))


# --------------------------------------------------------------------------
# fp16 / fp32 elementwise and glue
# --------------------------------------------------------------------------
def test_float_elementwise(backend):
    r = synth.Rng(synth.seed_for(10))
    n = 3001
    a32 = r.normal((n,), 0.0, 4.0)
    b32 = r.normal((n,), 0.0, 4.0)
    a16, b16 = synth.f16_bits(a32), synth.f16_bits(b32)
    ba, bb, ba16, bb16 = map(backend.from_numpy, (a32, b32, a16, b16))
    y32, y16 = backend.alloc(n * 4), backend.alloc(n * 2)
    for fn, ref in [(ops.add_f32, oracle.add_f32), (ops.mul_f32, oracle.mul_f32)]:
        fn(backend, ba, bb, y32, n)
        np.testing.assert_array_equal(backend.to_numpy(y32, np.float32, n), ref(a32, b32))
    for fn, ref in [(ops.add_fp16, oracle.add_fp16), (ops.mul_fp16, oracle.mul_fp16)]:
        fn(backend, ba16, bb16, y16, n)
        np.testing.assert_array_equal(backend.to_numpy(y16, np.uint16, n), ref(a16, b16))
    ops.relu_f32(backend, ba, y32, n)
    np.testing.assert_array_equal(backend.to_numpy(y32, np.float32, n), oracle.relu_f32(a32))
    ops.relu_fp16(backend, ba16, y16, n)
    np.testing.assert_array_equal(backend.to_numpy(y16, np.uint16, n), oracle.relu_fp16(a16))
    ops.sigmoid_f32(backend, ba, y32, n)
    np.testing.assert_allclose(backend.to_numpy(y32, np.float32, n), oracle.sigmoid_f32(a32), rtol=2e-7, atol=1e-7)
    ops.silu_fp16(backend, ba16, y16, n)
    assert rel_err(f16v(backend.to_numpy(y16, np.uint16, n)), f16v(oracle.silu_fp16(a16))) <= 1e-2
    ops.sigmoid_fp16(backend, ba16, y16, n)
    assert rel_err(f16v(backend.to_numpy(y16, np.uint16, n)), f16v(oracle.sigmoid_fp16(a16))) <= 1e-2


@pytest.mark.parametrize("case", [("u8", 32, (7, 5), (13, 11)), ("u8", 4, (20, 20), (40, 40)),
                                  ("u8", 128, (9, 12), (4, 7)), ("f16", 8, (6, 6), (12, 12)),
                                  ("f16", 6, (5, 9), (11, 3))])
def test_resize_nearest_scales_and_widths(backend, case):
    # 16-byte rows (u8 c=32/128, f16 c=8) and 4-byte rows, up and down.
    dt, c, (h, w), (ho, wo) = case
    r = synth.Rng(synth.seed_for(12 + c + h))
    if dt == "u8":
        x = r.integers((2, h, w, c), 0, 255).astype(np.uint8)
        dtype = ops.DTYPE_U8
    else:
        x = synth.f16_bits(r.normal((2, h, w, c), 0.0, 1.0))
        dtype = ops.DTYPE_F16
    bx = backend.from_numpy(x)
    by = backend.alloc(2 * ho * wo * c * x.itemsize)
    ops.resize_nearest_nhwc(backend, dtype, bx, by, 2, h, w, ho, wo, c)
    got = backend.to_numpy(by, x.dtype, (2, ho, wo, c))
    np.testing.assert_array_equal(got, oracle.resize_nearest(x, ho, wo))


def test_pool_resize_concat_split(backend):
    r = synth.Rng(synth.seed_for(11))
    x = synth.f16_bits(r.normal((2, 20, 20, 32), 0.0, 1.0))
    n, h, w, c = x.shape
    bx = backend.from_numpy(x)
    # SPPF pool: k5 s1 p2 (padded, extension) and the reference's unpadded 2x2 s2
    by = backend.alloc(x.nbytes)
    ops.maxpool2d_nhwc(backend, ops.DTYPE_F16, bx, by, n, h, w, c, 5, 5, 1, 1, (2, 2, 2, 2))
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, x.shape),
                                  oracle.maxpool2d_padded(x, (5, 5), (1, 1), (2, 2, 2, 2)))
    x32 = oracle.f16_to_f32(x)
    b32 = backend.from_numpy(x32)
    by = backend.alloc(n * 10 * 10 * c * 4)
    ops.maxpool2d_nhwc(backend, ops.DTYPE_F32, b32, by, n, h, w, c, 2, 2, 2, 2)
    np.testing.assert_array_equal(backend.to_numpy(by, np.float32, (n, 10, 10, c)),
                                  oracle.maxpool2d_f32(x32, (2, 2), (2, 2)))
    # nearest 2x
    by = backend.alloc(n * 40 * 40 * c * 2)
    ops.resize_nearest_nhwc(backend, ops.DTYPE_F16, bx, by, n, h, w, 40, 40, c)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, (n, 40, 40, c)), oracle.resize_nearest(x, 40, 40))
    # concat / split along channels
    parts = [x[..., :8].copy(), x[..., 8:24].copy(), x[..., 24:].copy()]
    bparts = [backend.from_numpy(p) for p in parts]
    by = backend.alloc(x.nbytes)
    ops.concat_channels_nhwc(backend, ops.DTYPE_F16, bparts, [8, 16, 8], by, n * h * w)
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint16, x.shape), oracle.concat_channels(parts))
    outs = [backend.alloc(p.nbytes) for p in parts]
    ops.split_channels_nhwc(backend, ops.DTYPE_F16, bx, outs, [8, 16, 8], n * h * w)
    for o, p, q in zip(outs, parts, oracle.split_channels(x, [8, 16, 8])):
        np.testing.assert_array_equal(backend.to_numpy(o, np.uint16, p.shape), q)
    # u8 padded maxpool
    xq = r.integers((1, 9, 11, 16), 0, 255).astype(np.uint8)
    bq = backend.from_numpy(xq)
    by = backend.alloc(xq.nbytes)
    ops.maxpool2d_nhwc(backend, ops.DTYPE_U8, bq, by, 1, 9, 11, 16, 5, 5, 1, 1, (2, 2, 2, 2))
    np.testing.assert_array_equal(backend.to_numpy(by, np.uint8, xq.shape),
                                  oracle.maxpool2d_padded(xq, (5, 5), (1, 1), (2, 2, 2, 2)))
