import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_package():
    import __graft_entry__
    return __graft_entry__.import_package()


def to_device(x: np.ndarray, device):
    """BF16 bits (uint16 numpy) -> torch.bfloat16 tensor on `device`."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).to(device)


def to_host_bits(t) -> np.ndarray:
    """torch.bfloat16 tensor -> BF16 bits (uint16 numpy)."""
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def gpu_runner(pkg):
    """The HIP library on cuda:0.  Fails (never skips) when either is missing."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    name = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    assert name == "gfx950", f"expected gfx950, found {name}"
    return pkg.Runner()
