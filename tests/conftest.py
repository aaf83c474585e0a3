import os
import sys

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(__file__))

import pytest  # noqa: E402
from hypothesis import settings  # noqa: E402

settings.register_profile("default", deadline=None, max_examples=40)
settings.register_profile("thorough", deadline=None, max_examples=400)
settings.load_profile(os.environ.get("HYPOTHESIS_PROFILE", "default"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle
    oracle._load()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exactattention_amd import hip
    hip.load()  # raises when the library is missing: no silent fallback
    return torch.device("cuda:0")
