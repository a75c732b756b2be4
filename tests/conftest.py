import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    # GPU tests never silently pass on a CPU-only machine: they are skipped
    # here only when the user deselects them (-m "not gpu"); when selected
    # without a GPU they fail in the fixture below.
    pass


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    from agpt_amd import _native
    _native.attn_lib()  # fails loudly if the HIP library is missing
    return torch.device("cuda:0")
