import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
for path in (REPO, REPO / "flash-attention-lab_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

from flash_lab import ops  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the HIP library")
    config.addinivalue_line("markers", "slow: large shapes (S >= 4096 or B*H >= 64)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip_gpu = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip_gpu)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


@pytest.fixture(autouse=True, scope="session")
def _no_tf32():
    # fp32 baselines must really be fp32.
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False


@pytest.fixture
def knobs():
    """The HIP library's routing knobs (flash_lab._hip.set_knob) for one test: every knob is
    restored to the value it had before the test when the test ends."""
    from flash_lab import _hip

    saved = {name: _hip.get_knob(name) for name in _hip.KNOBS}
    yield _hip.set_knob
    for name, value in saved.items():
        _hip.set_knob(name, value)


@pytest.fixture(scope="session")
def flash_ops():
    """torch.ops.flash_lab, failing loudly if a GPU is present but the HIP library did not load."""
    if not ops.HAS_EXTENSION:
        pytest.fail(f"a GPU is available but the HIP library did not load: {ops.EXTENSION_ERROR}")
    return torch.ops.flash_lab
