"""C++ host classes that need a GPU (tests/cpp/test_device.cpp): the device
arena with the reference's test_arena checks (tests/test_kernels.cu:510-533),
alignment, nested scopes, moves, and copies through the memory it hands out."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parent.parent


def test_device_arena():
    subprocess.run(["make", "-s", "-C", str(REPO / "tests" / "cpp")], check=True)
    out = subprocess.run([str(REPO / "tests" / "cpp" / "build" / "test_device")], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    assert "all device checks passed" in out.stdout
