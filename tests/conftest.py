import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (runs through the HIP C-ABI)')


@pytest.fixture(scope='session')
def golden():
    import numpy as np
    return np.load(ROOT / 'tests' / 'golden' / 'triton_vectors.npz')


@pytest.fixture(scope='session')
def dev():
    import torch
    if not torch.cuda.is_available():
        if Path('/dev/kfd').exists():
            pytest.fail('a ROCm device node exists but torch sees no GPU')
        pytest.skip('no GPU in this container')
    return torch.device('cuda:0')
