import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden" / "tiny_llama_fixture.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def golden():
    z = np.load(GOLDEN)
    data = {k: z[k] for k in z.files}
    import json

    data["config"] = json.loads(bytes(data["config"]).decode())
    return data


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def backend():
    from fracture_amd import HipBackend

    b = HipBackend(0)
    yield b
    b.close()


def close(actual, expected, rtol, atol):
    """The reference's comparison rule: |a - e| <= atol + rtol * |e|
    (tests/validation/src/tensor_compare.rs:291-292)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    return np.abs(a - e) <= atol + rtol * np.abs(e)


def assert_close(actual, expected, rtol, atol, what=""):
    ok = close(actual, expected, rtol, atol)
    if not ok.all():
        a = np.asarray(actual, dtype=np.float64)
        e = np.asarray(expected, dtype=np.float64)
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(
            f"{what}: {len(bad)}/{ok.size} elements outside atol={atol} rtol={rtol}; first at {i}: "
            f"got {a[i]!r} expected {e[i]!r}; max abs err {np.max(np.abs(a - e)):.3g}")
