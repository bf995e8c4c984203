import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "im-not-llm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

# Reference checkout: read only by CPU tests that regenerate or cross-check
# fixtures; GPU tests never touch it.
REFERENCE = Path(os.environ.get("INL_REFERENCE", "/root/reference"))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def inl():
    import inl_hip
    return inl_hip
