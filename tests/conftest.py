import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, 'musc-gpu_amd')):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, 'tests', 'golden')


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (ROCm GPU) and the built libmusc_hip.so')
    config.addinivalue_line('markers', 'slow: CPU test that takes more than a few seconds')


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available() and torch.version.hip is not None
    except Exception:
        return False


@pytest.fixture(scope='session')
def device():
    import torch
    if not gpu_available():
        pytest.fail('GPU test selected but no ROCm GPU is visible')
    return torch.device('cuda:0')


@pytest.fixture(scope='session')
def golden():
    import numpy as np

    def load(name):
        with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as f:
            return {k: f[k] for k in f.files}
    return load
