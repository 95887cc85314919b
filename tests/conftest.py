import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "stream-pt_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


@pytest.fixture(scope="session")
def O():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu_ctx():
    import torch

    import spt

    if not torch.cuda.is_available():
        pytest.fail("a gpu-marked test ran without a GPU")
    torch.cuda.set_device(0)
    ctx = spt.Context(0, torch.cuda.current_stream().cuda_stream)
    yield ctx
    ctx.close()
