"""The oracle still reproduces every committed golden fixture bit for bit
(tests/golden/*.npz, written by tests/golden/make_golden.py), so the fixtures
the GPU tests compare against stay tied to the pinned oracle."""
import importlib.util
import os

import numpy as np
import pytest

from helpers import GOLDEN

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_fixture_reproduces(name):
    stored = np.load(os.path.join(GOLDEN, name + ".npz"))
    fresh = make_golden.FIXTURES[name]()
    assert sorted(stored.files) == sorted(fresh)
    for k in stored.files:
        a, b = stored[k], np.asarray(fresh[k])
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert a.tobytes() == b.tobytes(), f"{name}.{k} differs from the oracle"
