import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skips GPU tests on a host without a GPU; on a GPU host the native
    library must load (no fallback path exists)."""
    if not _gpu_available():
        pytest.skip("no GPU on this host")
    from speculative_decode_engine_amd import _native
    _native.load()
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def oracle():
    from oracle import paged_kv
    paged_kv.lib()
    return paged_kv


def case_banner(*parts) -> None:
    """Prints (flushed) what a GPU test is about to run, so a failing run
    names its case even if the process dies."""
    print("[case]", *parts, flush=True)
    sys.stdout.flush()
    os.environ.get("PYTEST_CURRENT_TEST")
