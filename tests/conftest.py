from __future__ import annotations

import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm device and the built libintentir_hip.so")


def hip_ready() -> bool:
    """A ROCm device is visible (GPU tests fail loudly if the library is then missing)."""
    if os.environ.get("IHIP_FORCE_NO_GPU"):
        return False
    try:
        import torch
    except ImportError:
        return False
    return bool(torch.cuda.is_available())


@pytest.fixture(scope="session")
def hip():
    """Loaded C-ABI library; skips the test when no ROCm device is visible."""
    if not hip_ready():
        pytest.skip("no ROCm device")
    from intent_ir_amd.runtime import load_library

    return load_library()
