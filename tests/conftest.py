import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "delta-attention_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a GPU is present; fail loudly if the library is missing."""
    if not gpu_available():
        pytest.skip("no GPU")
    from delta_attention import _lib
    _lib.lib()  # raises ExtensionMissing when the HIP library is not built
    return True


@pytest.fixture(params=[32, 64], ids=["rows32", "rows64"])
def rows_per_wave(request, gpu):
    """Run the test with each tile shape of the head_dim-128 key-sparse
    launches (32 or 64 query rows per wave), restoring the previous one."""
    from delta_attention import ops
    prev = ops.set_sparse_rows_per_wave(request.param)
    yield request.param
    ops.set_sparse_rows_per_wave(prev)
