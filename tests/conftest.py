import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built extension")


@pytest.fixture(scope="session")
def fa():
    """The drop-in module, on a GPU.  Fails (not skips) if the native build is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import flash_attn_v100

    return flash_attn_v100
