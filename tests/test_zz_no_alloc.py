"""GPU: mi_mul_mat_q8_0_noalloc (the library's static per-GPU scratch, no
workspace argument) against mi_mul_mat_q8_0 with a workspace of its own, two
calls in a row with the second on a smaller input, through the C ABI.
Bar, written here: the same kernels on the same inputs, so y is bit-identical
to the workspace entry point's (which the matmul tests check against the
oracle); the second call must not see anything the first left in the scratch.
"""
import ctypes

import numpy as np
import pytest
from helpers import to_dev, to_np
from oracle import oracle as orc

from acestep_ops import _lib, ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu


def _case(n, k, m, seed):
    r = np.random.default_rng(seed)
    w = orc.quantize_q8_0(r.standard_normal((n, k)).astype(np.float32))
    x = r.standard_normal((m, k)).astype(np.float32)
    return ops.q8_0_repack(ops.Q8(to_dev(w))), to_dev(x)


@pytest.mark.parametrize("first,second", [
    ((2560, 9728, 8), (1000, 2560, 2)),    # decode GEMV with split partials, then a smaller one
    ((1536, 2048, 96), (300, 1024, 3)),    # matrix kernel (prefill rows), then a split decode GEMV
])
def test_noalloc_matches_workspace_entry(dev, first, second):
    for i, (n, k, m) in enumerate((first, second)):
        print(f"mul_mat_q8_0_noalloc call {i}: n={n} k={k} m={m}", flush=True)
        wr, dx = _case(n, k, m, seed=n + k + m)
        y_ws = to_np(ops.mul_mat_q8_0(wr, dx))
        y_na = DTensor.empty((m, n), "f32")
        ops.mul_mat_q8_0_noalloc(wr, dx, out=y_na)
        assert np.array_equal(to_np(y_na), y_ws), f"call {i}"


def test_noalloc_rejects_oversized_call(dev):
    """a product whose scratch exceeds the static array: MI_ERR_SCRATCH, nothing launched"""
    wr, _ = _case(64, 8192, 1, seed=3)
    x = DTensor.empty((8192, 8192), "f32")  # 64 MiB of quantized x
    y = DTensor.empty((8192, 64), "f32")
    assert ops.mul_mat_q8_0_workspace(wr, x) > _lib.NOALLOC_SCRATCH_BYTES
    rc = _lib.load().mi_mul_mat_q8_0_noalloc(ctypes.c_void_p(wr.data.ptr), wr.k, wr.n, ctypes.byref(ops.desc(x)),
                                             ctypes.byref(ops.desc(y)), None)
    assert rc == -10
