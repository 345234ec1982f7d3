import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    import geoembodied  # noqa: F401
    from gdl_amd import _native
    assert _native.loaded(), f"HIP library not loaded from {_native.library_path()}"
    print(f"[gpu] {torch.cuda.get_device_name(0)} | {_native.build_info()}", flush=True)
    return torch.device("cuda:0")
