import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: larger CPU case")


def load_package():
    """The product package (its directory name is not a Python identifier)."""
    return importlib.import_module("qr-contest_amd")


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def workloads(pkg):
    return importlib.import_module("qr-contest_amd.workloads")
