import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "llm-compressor_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmi355q.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    from llmcompressor_amd import _lib

    _lib.load_library()
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible ROCm device")
    return torch.device("cuda:0")
