import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen38-flash-next-b70-offload_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(autouse=True)
def _device_status_ok(request):
    """After every GPU test: no bounded wait of a decode kernel timed out (exl3_device_status flags4[0] == 0). A
    timeout means some output was computed from incomplete data, whatever the test itself compared."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import ctypes

    import torch
    from exl3xpu import capi
    if not torch.cuda.is_available():
        return
    flags = (ctypes.c_int32 * 4)()
    capi.check(capi.lib().exl3_device_status(flags, torch.cuda.current_stream().cuda_stream), "device status")
    assert flags[0] == 0, f"{flags[0]} bounded waits of the decode kernels timed out during {request.node.name}"
