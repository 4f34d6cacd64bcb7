import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE = ROOT / 'torch-intel-npu_amd'
for path in (ROOT, PACKAGE):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (ROCm device) and the built HIP library')


@pytest.fixture(scope='session')
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip('no ROCm device')
    import lowbit_hip
    lowbit_hip.library()  # fail loudly if the HIP library is missing
    return torch.device('cuda:0')


def announce(*parts):
    """Print and flush a line naming the GPU case about to run."""
    print('[case]', *parts, flush=True)
