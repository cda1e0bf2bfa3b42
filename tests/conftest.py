import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rust-ppocrv6_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

REFERENCE = "/root/reference"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure); built on demand where a compiler exists."""
    from oracle import oracle as o
    if not os.path.exists(o.LIB_PATH):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
    o.lib()
    return o


@pytest.fixture(scope="session")
def rh():
    """The product package (HIP library through its C ABI)."""
    import ppocr_rechead
    ppocr_rechead._lib.lib()
    return ppocr_rechead


def reference_available():
    return os.path.isdir(os.path.join(REFERENCE, "src"))


def rust_pattern(n, f, scale=1.0, offset_mod=None):
    """The reference tests' deterministic inputs: f(i * step) computed in f32."""
    i = np.arange(n, dtype=np.float32)
    return f(i).astype(np.float32) * np.float32(scale)
