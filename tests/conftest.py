"""Shared test setup.

Markers: tests that need the MI355X are marked `gpu`; everything else runs
on the CPU.  GPU tests talk to the library only through its C ABI (via the
ctypes binding in flash_deepseek_amd) and check it against the C
restatement under oracle/.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    return O


@pytest.fixture(scope="session")
def fdm():
    """The initialised library on cuda:0 (GPU tests only)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import flash_deepseek_amd as F
    F.init(0)
    return F


@pytest.fixture(autouse=True)
def _kernel_waits_completed(request):
    """After every test that used the library: no wait inside a layer kernel
    gave up during it (fdm_stream_sync reports such a call once)."""
    yield
    if "fdm" in request.fixturenames:
        request.getfixturevalue("fdm").sync()


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "quant_golden.npz")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
