"""The C ABI library: loads, exports every function include/dw_hip.h declares,
and reports errors through status codes (no compute without a GPU here)."""
import ctypes as C

import pytest

from dragonwing_edge_rs_amd import _lib


def test_library_exports_every_header_symbol():
    names = _lib.header_symbols()
    assert len(names) > 60
    assert _lib.missing_exports() == []


def test_signature_table_covers_header():
    assert set(_lib.header_symbols()) == set(_lib.SIGNATURES)


def test_backend_create_without_device_fails_cleanly():
    lib = _lib.load()
    h = C.c_void_p()
    rc = lib.dw_hip_backend_create(99, C.byref(h))
    assert rc == -1
    assert b"no HIP device" in lib.dw_last_error() or b"hip" in lib.dw_last_error().lower()


def test_null_arguments_are_errors():
    lib = _lib.load()
    assert lib.dw_hip_backend_create(0, None) == -4
    assert lib.dw_hip_upload(None, None, None, 0) == -4
    assert lib.dw_hip_buffer_len_bytes(None) == 0
    lib.dw_hip_buffer_free(None)  # no-op
