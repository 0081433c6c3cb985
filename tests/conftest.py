import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "ai-engine_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests run the HIP path and nothing else: no GPU is a failure."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    import pagedkv
    pagedkv.lib()  # fails loudly if libpagedkv.so is missing
    return torch.device("cuda", 0)
