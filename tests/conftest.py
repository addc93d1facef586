import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gpu_ready() -> bool:
    import torch
    if not torch.cuda.is_available():
        return False
    from diffucore_amd import _lib
    return _lib.device_is_gfx950(torch.cuda.current_device())


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; the HIP library must load (no fallback)."""
    import torch
    from diffucore_amd import _lib
    if not gpu_ready():
        pytest.skip("needs a gfx950 GPU")
    _lib.require()
    return torch.device("cuda", torch.cuda.current_device())
