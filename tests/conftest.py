import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built libnq_attn.so")
    config.addinivalue_line("markers", "slow: full-size configuration check")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from nano_qwen_amd._lib import lib
    lib()  # raises if the library is missing: no silent fallback
    return torch.device("cuda:0")
