import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


def _torch_gpu():
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 with libfmx loaded. Skips only where no GPU exists at all; on a
    GPU host a missing libfmx.so is an error, not a skip."""
    if not _torch_gpu():
        pytest.skip("no GPU in this environment")
    import torch
    from freemoe_amd import fmx
    fmx.lib()
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ref_lib():
    import fmoracle
    if not fmoracle.ref_available():
        pytest.skip("oracle/_ref not built (needs the FreeMoe tree at build time)")
    return fmoracle.ref()


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    """Names the GPU case on stdout before it runs, so a run that dies on the
    device still says which case it was in."""
    if request.node.get_closest_marker("gpu") is not None:
        sys.stdout.write(f"\n[gpu-case] {request.node.nodeid}\n")
        sys.stdout.flush()
    yield
