import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """The GPU test device. Skips without a GPU unless TQ_REQUIRE_GPU=1, which turns the skip into a
    failure (as the reference's TETRAEDER_REQUIRE_GPU does for its gpu_ tests)."""
    if not _gpu_available():
        if os.environ.get("TQ_REQUIRE_GPU") == "1":
            pytest.fail("TQ_REQUIRE_GPU=1 but no GPU is visible")
        pytest.skip("skip: no GPU visible")
    import torch
    from tetraeder_amd import _lib
    _lib.lib()  # the HIP library must load; there is no fallback
    return torch.device("cuda:0")
