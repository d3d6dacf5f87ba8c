import pathlib
import sys

import numpy as np
import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
for p in (REPO / "mlvc.cpp_amd" / "python", REPO / "oracle", REPO / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

# Parity bar of the FP16 path: relative to the oracle output RMS.
MAX_REL = 1e-2
MEAN_REL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels through the C ABI on an MI355X")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def assert_parity(got, want, what=""):
    import mlvc_oracle

    st = mlvc_oracle.parity_stats(got, want)
    assert st["finite"], f"{what}: non-finite output"
    assert st["max_rel"] <= MAX_REL and st["mean_rel"] <= MEAN_REL, f"{what}: {st}"
    return st
