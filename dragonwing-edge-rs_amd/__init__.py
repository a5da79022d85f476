"""dragonwing-edge-rs MI355X backend — Python host mirror of the C ABI.

Mirrors the reference's Rust surface so tests read like its own:

* :class:`Backend` — ``dragonwing_core::Backend`` (name / alloc / upload /
  download / synchronize), ``crates/dragonwing-core/src/backend.rs:127-199``.
* :mod:`.ops` — free op functions taking the backend, as
  ``dragonwing_vulkan::ops`` (``crates/dragonwing-vulkan/src/ops.rs``).
* :class:`.graph.Graph` / :class:`.graph.HipGraphRuntime` — ``Graph`` and
  ``VulkanGraphRuntime`` (``crates/dragonwing-onnx/src/vulkan_runtime.rs``).

All compute runs in libdwhip.so (HIP kernels for gfx950); importing this
package on a machine without the built library raises on first use.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import (RELEASE_BACKEND, RELEASE_BUFFER, HipError, check, load, native_calls_allowed,
                   release_all, track)

__all__ = ["Backend", "Buffer", "HipError", "load", "release_all", "BUFFER_STORAGE"]

BUFFER_STORAGE = 0


class Buffer:
    """A device byte buffer (``BackendBuffer``).  Freed by :meth:`free` or GC."""

    def __init__(self, backend: "Backend", handle: int, len_bytes: int):
        self._backend = backend
        self._h = handle
        self._len = len_bytes
        track(self, RELEASE_BUFFER)

    @property
    def handle(self) -> int:
        if self._h is None:
            raise HipError(-4, "buffer already freed")
        return self._h

    def len_bytes(self) -> int:
        return self._len

    def device_ptr(self) -> int:
        return load().dw_hip_buffer_device_ptr(self.handle)

    def free(self) -> None:
        # The C buffer holds its backend (reference-counted there), so it is
        # freed even after the Python Backend was closed.
        if self._h is not None:
            load().dw_hip_buffer_free(self._h)
        self._h = None

    _release = free

    def __del__(self):
        try:
            if native_calls_allowed():
                self.free()
        except Exception:
            pass


class Backend:
    """The HIP backend on one gfx950 device (one stream)."""

    def __init__(self, device: int = 0):
        lib = load()
        h = C.c_void_p()
        check(lib.dw_hip_backend_create(device, C.byref(h)))
        self._h = h.value
        track(self, RELEASE_BACKEND)

    @property
    def handle(self) -> int:
        return self._h

    def name(self) -> str:
        return load().dw_hip_backend_name(self._h).decode()

    def alloc(self, len_bytes: int, kind: int = BUFFER_STORAGE) -> Buffer:
        h = C.c_void_p()
        check(load().dw_hip_alloc(self._h, int(len_bytes), kind, C.byref(h)))
        return Buffer(self, h.value, int(len_bytes))

    def upload(self, dst: Buffer, src) -> None:
        data = np.ascontiguousarray(src)
        check(load().dw_hip_upload(self._h, dst.handle, data.ctypes.data, data.nbytes))

    def download(self, src: Buffer, dst: np.ndarray) -> None:
        if not dst.flags["C_CONTIGUOUS"]:
            raise ValueError("destination must be contiguous")
        check(load().dw_hip_download(self._h, src.handle, dst.ctypes.data, dst.nbytes))

    def synchronize(self) -> None:
        check(load().dw_hip_synchronize(self._h))

    # numpy conveniences ----------------------------------------------------
    def from_numpy(self, arr) -> Buffer:
        a = np.ascontiguousarray(arr)
        buf = self.alloc(a.nbytes)
        self.upload(buf, a)
        return buf

    def to_numpy(self, buf: Buffer, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        self.download(buf, out)
        return out

    def close(self) -> None:
        if self._h is not None:
            load().dw_hip_backend_destroy(self._h)
            self._h = None

    _release = close

    def __del__(self):
        try:
            if native_calls_allowed():
                self.close()
        except Exception:
            pass
