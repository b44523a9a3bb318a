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


@pytest.fixture(autouse=True)
def _output_guards(request):
    """Every workspace a GPU test makes allocates its outputs between guard regions (4 KiB of a
    fill byte on both sides, outside the registered buffer: the reference's poison guards,
    tests/metal/twin.hpp:42-66). After the test, each workspace's guards must be untouched."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    lay = ge.load_package().layer
    classes = (lay.LayerWorkspace, lay.PromptWorkspace, lay.DecodeWorkspace)
    originals = {c: c.__init__ for c in classes}
    made = []

    def wrap(orig):
        def init(self, *a, **k):
            orig(self, *a, **k)
            made.append(self)
        return init

    for c in classes:
        c.__init__ = wrap(originals[c])
    try:
        yield
    finally:
        for c in classes:
            c.__init__ = originals[c]
    import torch
    torch.cuda.synchronize()
    for ws in made:
        bad = ws.check_guards()
        assert not bad, f"{type(ws).__name__} {ws.cfg.name}: guard bytes written around output buffers {bad}"
