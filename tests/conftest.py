import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# Keep CPU oracle runs bounded and deterministic in thread count.
import torch  # noqa: E402

torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built native library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail (not skip) when it or the library is missing."""
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    arch = torch.cuda.get_device_properties(0).gcnArchName
    assert arch.startswith("gfx950"), f"expected gfx950, found {arch}"
    from kernelfuser_amd import _lib
    _lib.load()
    return torch.device("cuda:0")
