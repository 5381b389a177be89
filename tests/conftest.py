import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs on the GPU box")


@pytest.fixture(scope="session")
def hip():
    """The backend, set up on a real device. Skips only when no device is
    visible (SetupError::NoDevice); every other setup failure fails the test,
    as the reference's device() helper does (src/backend/cuda/tests/cuda_tests.rs:15-28)."""
    from poorgrad_amd import _native as n

    code = n.status()
    if code == n.NO_DEVICE:
        pytest.skip("no HIP device visible")
    assert code == n.OK, f"backend setup failed: {n.status_reason()}"
    import torch

    assert torch.cuda.is_available()
    return n


def banner(text: str) -> None:
    """Names the case on stdout before a GPU step (flushed), so a run that
    ends abruptly still shows what it was doing."""
    print(f"[case] {text}", flush=True)
