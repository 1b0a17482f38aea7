import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle

    pyoracle.build()
    return pyoracle


@pytest.fixture(scope="session")
def sampler():
    """One device sampler for the whole GPU session (fails loudly if the
    library or the GPU is missing)."""
    import torch

    import tinygpt_amd as tg

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    s = tg.Sampler(device=0, max_batch=1024, max_vocab=152064, max_hist=1024)
    yield s
    s.close()
