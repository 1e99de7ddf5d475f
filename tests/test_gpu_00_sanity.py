"""First GPU test: the runtime the library runs on, a host/device round trip
and one tiny op. Runs before the rest (file name) so `-x` stops early on a
broken setup."""
import numpy as np
import pytest

from helpers import to_dev, to_np

from acestep_ops import device, ops

pytestmark = pytest.mark.gpu


def test_runtime_and_roundtrip(dev):
    v = device.runtime_version()
    print("HIP runtime version", v, "devices", device.device_count(), flush=True)
    assert v > 0
    a = np.arange(4096, dtype=np.float32)
    assert np.array_equal(to_np(to_dev(a, dev)), a)
    big = np.random.default_rng(0).standard_normal(3 << 20).astype(np.float32)  # 12 MB
    assert np.array_equal(to_np(to_dev(big, dev)), big)


def test_tiny_add(dev):
    a = np.arange(64, dtype=np.float32).reshape(4, 16)
    b = np.ones((4, 16), np.float32)
    y = to_np(ops.add(to_dev(a, dev), to_dev(b, dev)))
    device.synchronize()
    assert np.array_equal(y, a + b)
