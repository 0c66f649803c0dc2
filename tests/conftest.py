import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vpipe-ming-image_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    """One context on cuda:0 for the GPU tests. The product library must be
    built: a missing library fails loudly instead of skipping."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ming_dit_amd as m
    c = m.Ctx(0)
    yield c
    c.close()
