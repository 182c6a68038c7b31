import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# the package lives in kiln-compiler_amd/; tests/models is importable as `models`;
# the oracle package is at the repo root.
for p in (os.path.join(ROOT, "kiln-compiler_amd"), os.path.dirname(os.path.abspath(__file__)), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU); run with -m gpu")


@pytest.fixture(autouse=True)
def _gpu_tests_run_on_the_gpu(request):
    # the host interpreter (KILN_HIP_INTERPRET) is a CPU test instrument; a
    # GPU-marked test must exercise the HIP path
    if request.node.get_closest_marker("gpu") is not None:
        from kiln.hip.interpret import refuse

        refuse(request.node.nodeid)
    yield


@pytest.fixture(autouse=True)
def _deterministic():
    torch.manual_seed(0)
    yield


@pytest.fixture(autouse=True)
def private_cache(tmp_path, monkeypatch):
    monkeypatch.setenv("KILN_CACHE_DIR", str(tmp_path))
    yield
