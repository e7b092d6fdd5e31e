"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (run with `-m gpu` on the GPU box); all
others run on any host (`-m "not gpu"`).
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "project-ia_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu)")


def pytest_runtest_setup(item):
    # Print the case name before each GPU test so a run that ends the box
    # still shows which case it was in.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)


@pytest.fixture(scope="session")
def qa():
    import qorus_amd
    if not qorus_amd.gpu_available():
        pytest.fail("no usable GPU: " + qorus_amd.lib().qh_last_error().decode())
    return qorus_amd


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    return oracle
