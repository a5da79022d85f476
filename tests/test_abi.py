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


def test_op_params_layout_matches_library():
    # dw_graph_add_op copies a whole dw_op_params: the binding's struct must
    # be exactly the library's.
    assert C.sizeof(_lib.DwOpParams) == _lib.load().dw_op_params_size()


def test_exit_releases_handles_in_order(tmp_path):
    # At interpreter exit live handles are released runtimes -> buffers ->
    # backends -> graphs, and finalizers make no native call afterwards.
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    script = tmp_path / "exit_order.py"
    script.write_text(f"""
import sys
sys.path.insert(0, {str(root)!r})
import __graft_entry__
__graft_entry__.import_pkg()
from dragonwing_edge_rs_amd import _lib
from dragonwing_edge_rs_amd.graph import Graph
order = []
class Fake:
    def __init__(self, tag, kind):
        self.tag = tag
        _lib.track(self, kind)
    def _release(self):
        order.append(self.tag)
objs = [Fake("graph", _lib.RELEASE_GRAPH), Fake("backend", _lib.RELEASE_BACKEND),
        Fake("buffer", _lib.RELEASE_BUFFER), Fake("runtime", _lib.RELEASE_RUNTIME)]
g = Graph()  # a real host-only handle, destroyed by the hook
keep = [g]
_lib.release_all()
assert order == ["runtime", "buffer", "backend", "graph"], order
assert g.handle is None
assert not _lib.native_calls_allowed()
print("ok")
""")
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip().endswith("ok")
