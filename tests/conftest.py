import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libaegkv kernels)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    if not o.LIB.exists():
        o.build()
    return o


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def load(name):
        return np.load(GOLDEN / name, allow_pickle=False)

    return load


@pytest.fixture(scope="session")
def aegkv_lib():
    """The built C-ABI library (compiled here if the tree has none yet)."""
    from aegaeon_amd import _lib, build

    if not _lib.LIB_PATH.exists():
        build.build()
    return _lib.load()


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from aegaeon_amd import _lib

    _lib.load()  # fail loudly, never fall back, if the HIP library is missing
    return torch.device("cuda:0")
