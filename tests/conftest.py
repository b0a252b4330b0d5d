import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")
    importlib.import_module("tests._live").attach(config)


def pytest_sessionstart(session):
    """Builds the libraries once when the tree has none (a fresh checkout);
    a built tree is used as it is."""
    importlib.import_module("__graft_entry__").ensure_built()


@pytest.fixture(scope="session")
def mg():
    """The package (its directory name has hyphens, so import it by name)."""
    return importlib.import_module("minigpt-train-infra_amd")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def load(name):
        return np.load(ROOT / "tests" / "golden" / f"{name}.npz", allow_pickle=False)

    return load
