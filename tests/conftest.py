import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libkernrelay.so")
    config.addinivalue_line("markers", "slow: long-running (large shapes)")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Device guard for GPU tests: with a GPU present the library must load (no fallback)."""
    if not gpu_available():
        pytest.skip("no GPU visible")
    from kernrelay_amd import libapi
    libapi.lib()  # raises if the built library is missing
    return 0


@pytest.fixture(scope="session")
def workdir(tmp_path_factory):
    return tmp_path_factory.mktemp("kr")


def announce(msg):
    """Print (and flush) what a GPU step is about to run, so a run that dies
    still names its case."""
    print("[kr-test] " + msg, flush=True)
    sys.stdout.flush()
    sys.stderr.flush()
