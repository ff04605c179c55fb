import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU check")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from robolearn_amd import _native

    _native.load()
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _single_thread_cpu():
    import torch

    previous = torch.get_num_threads()
    torch.set_num_threads(int(os.environ.get("RL_TEST_THREADS", "4")))
    yield
    torch.set_num_threads(previous)
