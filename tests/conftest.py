"""pytest configuration: the `gpu` marker, import paths for the library's Python mirror and the CPU oracle."""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "xestrata-win_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libxsmoe.so")


@pytest.fixture(scope="session")
def xo():
    import xs_oracle
    xs_oracle.lib()
    return xs_oracle


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    g = ROOT / "tests" / "golden"
    return dict(np.load(g / "reference_vectors.npz")), dict(np.load(g / "seeded_inputs.npz"))


@pytest.fixture(scope="session")
def xm():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test without a GPU")
    import xsmoe
    xsmoe.lib()
    return xsmoe
