import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "mlir-gpu-kernel-compiler_amd"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libtjhip.so")


@pytest.fixture
def tj_env(monkeypatch, tmp_path):
    """Isolated cache dir and analytic tile choice (as the reference's tests do)."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    monkeypatch.setenv("TENSORJIT_CACHE_DIR", str(tmp_path / "cache"))
    yield tmp_path


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available() and torch.version.hip is not None
    except Exception:
        return False

