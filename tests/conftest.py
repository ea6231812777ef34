import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import __graft_entry__  # noqa: E402

PKG = __graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU oracle work of more than a few seconds")


@pytest.fixture(scope="session")
def pkg():
    return PKG


@pytest.fixture(scope="session")
def weights_dir(tmp_path_factory):
    """Synthetic Big-LaMa containers: `plain` (the BASELINE fixture, seed 0)
    and `cal` (the same weights with calibrated BN statistics)."""
    import oracle_api as O

    d = tmp_path_factory.mktemp("weights")
    plain = str(d / "w0.safetensors")
    PKG.host_api.synth_weights(plain, 0)
    cal = str(d / "w0cal.safetensors")
    O.calibrated_weights(plain, cal, 64)
    return {"plain": plain, "cal": cal}


@pytest.fixture(scope="session")
def engine(weights_dir):
    eng = PKG.hip_engine.Engine()
    store = PKG.host_api.Store(weights_dir["cal"])
    eng.load_weights(store)
    eng._cal_store = store
    yield eng
    eng.close()


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    n = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (n if n > 0 else 1.0))
