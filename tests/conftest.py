import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(ROOT, "tests", "golden", "golden.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def O():
    """The CPU oracle (checker)."""
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def mxq_lib():
    """libmxq.so loaded through its C ABI (built in-tree if absent)."""
    from wuxianhuabu_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from wuxianhuabu_amd import build
        build.build()
    return _lib.lib()


@pytest.fixture(scope="session")
def dev(mxq_lib):
    """cuda:0, for tests marked gpu. Skips only when no GPU is present; a GPU
    with a missing or broken libmxq fails in mxq_lib above."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")
