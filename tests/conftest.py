import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, HERE)
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "42-berlin-engine_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP product library)")


def golden(name):
    return np.load(os.path.join(HERE, "golden", f"{name}.npz"), allow_pickle=False)


@pytest.fixture(scope="session")
def orc():
    from oracle_bind import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle_bind import RefLib, ref_available
    if not ref_available():
        pytest.skip("compiled reference (oracle/_ref) not built here")
    return RefLib()


@pytest.fixture(scope="session")
def be():
    """The HIP product library on cuda:0 (GPU tests only)."""
    import be42
    lib = be42.load()
    if not lib.device_available():
        pytest.fail("no HIP device: GPU tests must run on an MI355X")
    lib.init(0)
    return lib


def rel_err(got, want):
    """max |got - want| / max |want| (normwise relative error)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.abs(want).max()
    return float(np.abs(got - want).max() / (den if den > 0 else 1.0))
