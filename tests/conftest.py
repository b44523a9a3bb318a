import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import __graft_entry__ as ge  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def pkg():
    return ge.load_package()


@pytest.fixture(scope="session")
def orc():
    return ge.load_oracle()


@pytest.fixture(scope="session")
def moe(pkg):
    return pkg.moe


@pytest.fixture(scope="session")
def layer(pkg):
    return pkg.layer


@pytest.fixture(scope="session")
def gpu_ctx(moe):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return moe.Context(0)


@pytest.fixture(scope="session")
def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream
