import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "hbd-acestep.cpp_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def _have_gpu() -> bool:
    return os.path.exists("/dev/kfd")


def pytest_collection_modifyitems(config, items):
    # Without a GPU device node (a machine with no GPU) GPU tests are skipped;
    # on a machine with a GPU they always run, so a broken device fails instead of skipping.
    if _have_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU device in this container")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    """Device 0 through the HIP runtime libmi_ops.so links (never torch's)."""
    assert "torch" not in sys.modules, "GPU tests must not share a process with torch's HIP runtime"
    from acestep_ops import device

    assert device.device_count() > 0, "GPU test on a box without a usable GPU"
    device.check(device.hip().hipSetDevice(0), "hipSetDevice")
    maps = [l.split()[-1] for l in open("/proc/self/maps") if "libamdhip64" in l]
    assert maps and all("torch" not in m for m in maps), f"unexpected HIP runtime: {set(maps)}"
    return 0
