import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) GPU and the built HIP library')


@pytest.fixture(scope='session')
def golden():
    import numpy as np
    return np.load(ROOT / 'tests' / 'golden' / 'tcq_format_golden.npz', allow_pickle=False)
