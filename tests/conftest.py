import os
import sys

import numpy as np
import pytest

# PyTorch-ROCm ships its own HIP runtime and loads it as "libamdhip64.so";
# libpokit_hip.so asks for soname "libamdhip64.so.7", which that copy also
# carries.  Importing torch first makes both share one runtime (one HSA
# instance per process); loading our library first would bring up a second.
try:
    import torch  # noqa: F401
except ImportError:
    torch = None

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libpokit_hip.so)")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def port():
    import oracle
    if not oracle.available("port"):
        oracle.build(reference=False)
    return oracle.Oracle("port")


@pytest.fixture(scope="session")
def hip():
    """One backend for the whole GPU session (a single process on the card)."""
    from pokitlms_amd.backend import HipBackend
    b = HipBackend(0)
    yield b
    b.close()


def normwise_rel(gpu, cpu) -> float:
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    scale = np.max(np.abs(cpu))
    return float(np.max(np.abs(gpu - cpu)) / (scale if scale > 0 else 1.0))
