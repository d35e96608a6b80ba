import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def dev():
    """The HIP device as a torch device; GPU tests fail loudly without one."""
    import torch

    import gpt_amd

    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    assert gpt_amd.device_ok(), "libgpt_hip_attn.so reports no usable HIP device"
    return torch.device("cuda:0")
