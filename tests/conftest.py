import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def hip():
    """The HIP library bound through ctypes (fails loudly when it is not built)."""
    import infengine_amd
    return infengine_amd


@pytest.fixture(scope="session")
def ctx():
    import torch
    from infengine_amd.engine import Context
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    c = Context(0, graph=False)
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.fixture(autouse=True)
def _gpu_stream(request):
    """GPU tests run torch and the library on the session context's stream."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    import torch
    import gpu_util
    c = request.getfixturevalue("ctx")
    torch.cuda.synchronize()
    torch.cuda.set_stream(c.stream)
    yield
    torch.cuda.synchronize()
    gpu_util.release()
