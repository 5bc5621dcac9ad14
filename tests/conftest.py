import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "gemma4-webgpu_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from g4attn import abi

    abi.load()
    abi.call("g4_set_device", 0)
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Name the case on stdout (flushed) before it touches the GPU."""
    print(f"[case] {msg}", flush=True)
