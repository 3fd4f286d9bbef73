import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


PREFILL_MAX_B, PREFILL_MAX_POS = 1300, 42000  # largest prefill chunk / window any test runs on the default stream


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    o.lib()
    return o


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    import qwengine_amd
    qwengine_amd.ops.lib()  # loud failure if the HIP library is missing
    # set-up of the drop-in prefill: the default stream's workspace, for every prefill the tests run on it
    qwengine_amd.ops.attn_prefill_reserve(PREFILL_MAX_B, PREFILL_MAX_POS)
    return torch.device("cuda:0")
