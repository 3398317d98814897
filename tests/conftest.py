import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = Path(__file__).resolve().parent / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def load_golden(name: str) -> dict:
    """Golden vectors written by tests/golden/make_golden.py, as CPU torch tensors
    (bf16 arrays restored from their stored bit patterns)."""
    data = np.load(GOLDEN / f"{name}.npz")
    out = {}
    for key in data.files:
        if key.endswith("__bf16"):
            continue
        arr = np.ascontiguousarray(data[key])
        if f"{key}__bf16" in data.files:
            out[key] = torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16)
        else:
            out[key] = torch.from_numpy(arr)
    return out


@pytest.fixture
def golden():
    return load_golden


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 with the HIP library loaded; skips only when no HIP device is visible."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from lightdelta_amd import _lib

    _lib.load()  # raises (fails the test) when the library is missing
    return torch.device("cuda:0")
