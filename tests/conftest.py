"""Test configuration: puts the repo root on sys.path, imports the backend
package (its directory name is not an identifier) and registers the `gpu`
marker.  CPU tests run everywhere; `-m gpu` tests need an MI355X."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.import_pkg()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def backend():
    import dragonwing_edge_rs_amd as dw

    be = dw.Backend(0)
    yield be
    be.close()


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before it runs, so a run that dies mid-test says which.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
