import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch.device("cuda", 0)


@pytest.fixture(params=[0, 1], ids=["tiles_auto", "tiles_256x256"])
def tile_policy(request, device):
    """Runs a GPU test with the S8 launches' own choice of tile geometry and
    again with 256 x 256 tiles forced for every GEMM launch (the automatic
    choice takes them only for launches that fill the device, which the
    small test shapes do not)."""
    from sandmuon_amd import _native
    prev = _native.s8_tile_geometry(request.param)
    try:
        yield request.param
    finally:
        _native.s8_tile_geometry(prev)
