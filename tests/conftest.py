import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(autouse=True)
def _no_kernel_error_bits(request):
    """Every GPU test starts with the kernels' sticky error bits clear and must end with
    them still clear: no bounded wait gave up and no index was clamped."""
    if "gpu" not in request.keywords or not torch.cuda.is_available():
        yield
        return
    from exactkv_amd import _lib, kernels
    kernels.error_bits(clear=True)
    yield
    bits = kernels.error_bits(clear=True)
    assert bits == 0, f"kernel error bits {bits:#x}: {_lib.describe_errors(bits)}"


def u16(t):
    """bf16 torch tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def same_bits(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))
