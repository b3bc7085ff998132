import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vc4-gles2-inference_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvgx's C-ABI)")


@pytest.fixture(scope="session")
def gpu():
    """A libvgx context on cuda:0.  Skips where there is no GPU; on a GPU host a
    missing libvgx is an error, never a silent fallback."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from vgx import gpu as vg
    g = vg.GPU(0)
    yield g
    torch.cuda.synchronize()
    g.close()
