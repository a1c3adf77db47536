import importlib.util
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))
if str(REPO / "tests") not in sys.path:
    sys.path.insert(0, str(REPO / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs through the C-ABI")
    config.addinivalue_line("markers", "slow: long CPU test (full-size oracle)")


def load_lcr():
    if "lcr_amd" in sys.modules:
        return sys.modules["lcr_amd"]
    spec = importlib.util.spec_from_file_location("lcr_amd", REPO / "llama-cuda-runtime_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["lcr_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def lcr():
    return load_lcr()


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.load()
    return oracle


@pytest.fixture(autouse=True)
def _release_device_buffers():
    yield
    import helpers
    helpers.release_all()


@pytest.fixture(scope="session")
def gpu(lcr):
    """Skips unless a HIP device is visible; the library must then be built."""
    lib = lcr.load_library()
    if lib.lcr_device_count() < 1:
        pytest.skip("no HIP device")
    return lib


@pytest.fixture(scope="session")
def full_ckpt(lcr, tmp_path_factory):
    """The benchmark's full-size Llama-3.2-1B-architecture checkpoint (seeded
    N(0, 0.02) bf16 weights), written once per test session."""
    d = tmp_path_factory.mktemp("full_model")
    lcr.write_synthetic_checkpoint(d, lcr.llama_config(), seed=lcr.WEIGHT_SEED)
    return d
