import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def tiny_stablelm():
    """The reference's tiny StableLM fixture (testdata/stablelm)."""
    from tinyoai_amd import weights
    config, tensors = weights.load_safetensors_dir(os.path.join(GOLDEN, "stablelm"))
    return weights.validate_stablelm_config(config), tensors
