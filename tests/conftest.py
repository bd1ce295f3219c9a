import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def olib():
    import oracle
    oracle.build()
    return oracle.lib()


@pytest.fixture(scope="session")
def gpu():
    """A context on cuda:0 ordered on torch's current stream."""
    import torch
    import hotarubi_amd as hb
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    ctx = hb.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    yield ctx
    ctx.close()
