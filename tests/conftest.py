import importlib
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (HIP device)')


@pytest.fixture(scope='session')
def pkg():
    return importlib.import_module('dcss-auto_amd')


@pytest.fixture(scope='session')
def golden():
    return ROOT / 'tests' / 'golden'
