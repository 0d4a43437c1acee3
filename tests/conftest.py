"""Shared test setup: import paths, the `gpu` marker, and the oracle fixtures.

The oracle (oracle/, test infrastructure) is built here if its shared library
is missing; on the GPU box the prebuilt files travel with the tree.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "contract-stablehlo-mlx_amd")
for p in (PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (runs through the HIP C-ABI)")


def _ensure_oracle():
    lib = os.path.join(ROOT, "oracle", "build", "liboracle.so")
    exe = os.path.join(ROOT, "oracle", "build", "ggml_oracle")
    if not (os.path.exists(lib) and os.path.exists(exe)):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
    return lib, exe


@pytest.fixture(scope="session")
def oracle():
    _ensure_oracle()
    import oracle_py
    return oracle_py


def _write_refs(tmp_path_factory, flavor):
    _, exe = _ensure_oracle()
    d = tmp_path_factory.mktemp(f"ref_{flavor}")
    subprocess.run([exe, str(d), "--flavor", flavor], check=True, capture_output=True)
    return str(d)


@pytest.fixture(scope="session")
def ref_pinned(tmp_path_factory):
    """Every ggml_ref case written by the oracle, pinned flavour."""
    return _write_refs(tmp_path_factory, "pinned")


@pytest.fixture(scope="session")
def ref_stock(tmp_path_factory):
    """Every ggml_ref case written by the oracle, stock flavour."""
    return _write_refs(tmp_path_factory, "stock")


@pytest.fixture(params=["graph", "replay"])
def graph_mode(request):
    """Compiled functions traced in the test either captured into a hipGraph
    ("graph": every trace) or re-issuing their recorded launches ("replay")."""
    import shlo_hip
    prev = shlo_hip.set_graph_min_ops(1 if request.param == "graph" else 1 << 30)
    yield request.param
    shlo_hip.set_graph_min_ops(prev)
