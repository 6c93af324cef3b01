import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "qwen-ascend_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _decode_flag_clear(request):
    """After every GPU test: no decode call on the device's shared counters
    array had a bounded wait time out."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    from qmoe import _lib
    import torch
    cnt = _lib._COUNTERS.get(("cuda", 0))
    if cnt is not None and torch.cuda.is_available():
        assert _lib.decode_status(cnt, clear=True) == 0, "a decode wait timed out during this test"
