"""Deterministic synthetic workloads.

The generator is the reference test LCG (``crates/dragonwing-test/src/generators.rs:19-34``):
``state = state * 6364136223846793005 + 1442695040888963407 (mod 2^64)`` and
``next_f32 = (state >> 40) / 2^24``, vectorised here by jumping ahead in
blocks (``state_{s+j} = a^j * state_s + c * (a^{j-1} + ... + 1)``).  Seeds
follow the harness convention ``0xDEAD_BEEF_CAFE_BABE + 12345 * index``
(``crates/dragonwing-test/src/harness.rs:35``, ``:105-106``).

Derived distributions (all from the same stream, in this order per call):
uniform ``a + u * (b - a)`` in f32; normal by Box-Muller on ``(1 - u1, u2)``;
integers ``floor(u * (hi - lo + 1)) + lo``; log-uniform
``exp(ln a + u * (ln b - ln a))`` in f64, rounded to f32.
"""
from __future__ import annotations

import numpy as np

A = 6364136223846793005
CINC = 1442695040888963407
MASK = (1 << 64) - 1
DEFAULT_SEED = 0xDEADBEEFCAFEBABE
_BLOCK = 1 << 14
_JUMP = None


def seed_for(index: int) -> int:
    return (DEFAULT_SEED + 12345 * index) & MASK


def _jump_tables():
    global _JUMP
    if _JUMP is None:
        a_pow = np.empty(_BLOCK, np.uint64)
        c_acc = np.empty(_BLOCK, np.uint64)
        ap, cs = 1, 0
        for j in range(_BLOCK):
            # state after j+1 steps from s: a^(j+1) * s + c * sum_{i<=j} a^i
            cs = (cs * A + CINC) & MASK
            ap = (ap * A) & MASK
            a_pow[j] = ap
            c_acc[j] = cs
        _JUMP = (a_pow, c_acc)
    return _JUMP


class Rng:
    """The reference LCG with a vectorised draw."""

    def __init__(self, seed: int):
        self.state = int(seed) & MASK

    def next_u64(self, n: int) -> np.ndarray:
        a_pow, c_acc = _jump_tables()
        out = np.empty(n, np.uint64)
        pos = 0
        s = np.uint64(self.state)
        with np.errstate(over="ignore"):
            while pos < n:
                k = min(_BLOCK, n - pos)
                blk = a_pow[:k] * s + c_acc[:k]
                out[pos:pos + k] = blk
                s = blk[-1]
                pos += k
        self.state = int(s)
        return out

    def f32(self, n: int) -> np.ndarray:
        """next_f32: (state >> 40) / 2^24 in [0, 1)."""
        return (self.next_u64(n) >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)

    def uniform(self, shape, lo: float, hi: float) -> np.ndarray:
        n = int(np.prod(shape))
        u = self.f32(n)
        lo32, hi32 = np.float32(lo), np.float32(hi)
        return (lo32 + u * (hi32 - lo32)).astype(np.float32).reshape(shape)

    def normal(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        n = int(np.prod(shape))
        u = self.f32(2 * n).astype(np.float64).reshape(n, 2)
        z = np.sqrt(-2.0 * np.log(1.0 - u[:, 0])) * np.cos(2.0 * np.pi * u[:, 1])
        return (mean + std * z).astype(np.float32).reshape(shape)

    def integers(self, shape, lo: int, hi: int) -> np.ndarray:
        """Uniform integers in [lo, hi] inclusive (int64)."""
        n = int(np.prod(shape))
        u = self.f32(n).astype(np.float64)
        return (np.floor(u * (hi - lo + 1)).astype(np.int64) + lo).reshape(shape)

    def log_uniform(self, shape, lo: float, hi: float) -> np.ndarray:
        n = int(np.prod(shape))
        u = self.f32(n).astype(np.float64)
        return np.exp(np.log(lo) + u * (np.log(hi) - np.log(lo))).astype(np.float32).reshape(shape)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits, round to nearest even (numpy's float16 cast)."""
    return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16_value(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, np.uint16).view(np.float16).astype(np.float32)


# --------------------------------------------------------------------------
# The single-op workloads (input tensors in the layouts the C ABI takes).
# --------------------------------------------------------------------------

def conv_f32_case(index: int = 0, n=1, c_in=64, c_out=64, h=56, w=56, k=3):
    """Conv2d fp32 + bias + ReLU: x, W uniform[-1,1], bias uniform[-0.1,0.1].

    x is generated NCHW and W as [Co][Ci][kh][kw] (the ONNX layouts), then
    permuted to NHWC / HWIO as convert_nchw_to_nhwc does.
    """
    r = Rng(seed_for(index))
    x_nchw = r.uniform((n, c_in, h, w), -1.0, 1.0)
    w_oihw = r.uniform((c_out, c_in, k, k), -1.0, 1.0)
    b = r.uniform((c_out,), -0.1, 0.1)
    return (np.ascontiguousarray(x_nchw.transpose(0, 2, 3, 1)),
            np.ascontiguousarray(w_oihw.transpose(2, 3, 1, 0)), b)


def qlinearconv_case(index: int = 1, n=32, h=80, w=80, c_in=128, c_out=256, k=3):
    """QLinearConv u8 x s8 -> u8: x u8 uniform {0..255}, W s8 uniform
    {-127..127} (generated [Co][kh][kw][Ci], stored HWIO), per-channel
    weight scales log-uniform [1e-3, 1e-2], bias int32 uniform
    [-4096, 4096]; x_scale 0.02 / zp 128, y_scale 0.05 / zp 128."""
    r = Rng(seed_for(index))
    x = r.integers((n, h, w, c_in), 0, 255).astype(np.uint8)
    w_ohwi = r.integers((c_out, k, k, c_in), -127, 127).astype(np.int8)
    ws = r.log_uniform((c_out,), 1e-3, 1e-2)
    bias = r.integers((c_out,), -4096, 4096).astype(np.int32)
    w_hwio = np.ascontiguousarray(w_ohwi.transpose(1, 2, 3, 0))
    return dict(x=x, w=w_hwio, w_scales=ws, bias=bias, x_scale=0.02, x_zp=128, y_scale=0.05, y_zp=128)


def dwconv_case(index: int = 2, n=32, c=384, h=40, w=40, k=3):
    """Depthwise 3x3 fp16 + bias + SiLU: x N(0,1), W N(0,0.1), bias N(0,0.1)."""
    r = Rng(seed_for(index))
    x = f16_bits(r.normal((n, h, w, c), 0.0, 1.0))
    wt = f16_bits(r.normal((k, k, c), 0.0, 0.1))
    b = f16_bits(r.normal((c,), 0.0, 0.1))
    return x, wt, b
