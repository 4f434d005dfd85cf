import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = Path(__file__).resolve().parent / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")
    config.addinivalue_line("markers", "slow: long-running statistical test")


def load_golden(name: str) -> dict:
    with np.load(GOLDEN / name) as z:  # allow_pickle stays False
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; GPU tests need the HIP library and a visible device."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from woodcock_amd import _lib

    _lib.lib()  # raises if libwoodcock_hip.so is missing: no fallback
    return torch.device("cuda", 0)
