import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

REFERENCE = Path("/root/reference")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; fails loudly (no CPU fallback) if the HIP library is absent."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import xtile_amd  # noqa: F401  (loads libxtile_amd.so)

    return torch.device("cuda:0")


def oracle_threads() -> int:
    return int(os.environ.get("XT_ORACLE_THREADS", min(16, os.cpu_count() or 1)))
