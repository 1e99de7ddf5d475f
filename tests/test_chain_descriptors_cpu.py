"""Host audit of the descriptors the DiT block test hands mi_dit_block_ops.

Runs without a GPU: the storage is a stand-in that only hands out disjoint
address ranges of the requested sizes. Every mi_tensor in the filled
MiDitBlockIO must address bytes inside the allocation it points into, and the
shape relations mi_dit_block_ops relies on (the same rows in every [H, S, N]
operand, one position per Q/K token, 2I -> I for SwiGLU, per-head CA views)
must hold. This is the host-side check the GPU test relies on before it
launches anything.
"""
import math

import numpy as np
import pytest

import dit_block_case
from dit_block_case import D, H, I, NH, NKV

from acestep_ops import _lib
from acestep_ops.device import DTYPES, DTensor


class _StandIn:
    """An allocation of `nbytes` at a fresh, page-separated fake address."""
    next_addr = 1 << 40

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = _StandIn.next_addr
        _StandIn.next_addr += (self.nbytes // 4096 + 2) * 4096
        ALLOCS.append(self)


ALLOCS = []


class _HostStorage:
    @staticmethod
    def empty(shape, dtype):
        return DTensor(_StandIn(math.prod(shape) * DTYPES[dtype][0]), shape, dtype)

    @staticmethod
    def up(a, dtype):
        dtype = dtype or {np.dtype(np.float32): "f32", np.dtype(np.int32): "i32"}[a.dtype]
        return DTensor(_StandIn(a.nbytes), a.shape, dtype)


def _span(t):
    """[lo, hi) bytes a ggml descriptor can address (0-element tensors address nothing)."""
    ne = [t.ne[i] for i in range(4)]
    if 0 in ne:
        return t.data, t.data
    es = 34 if t.type == _lib.Q8_0 else {_lib.F32: 4, _lib.I32: 4, _lib.BF16: 2, _lib.F16: 2}[t.type]
    n0 = ne[0] // 32 if t.type == _lib.Q8_0 else ne[0]
    hi = t.data + (n0 - 1) * t.nb[0] + sum((ne[d] - 1) * t.nb[d] for d in (1, 2, 3)) + es
    return t.data, hi


def _owner(addr):
    for a in ALLOCS:
        if a.ptr <= addr < a.ptr + max(a.nbytes, 1):
            return a
    return None


def _rows(t):
    return t.ne[1] * t.ne[2] * t.ne[3]


@pytest.mark.parametrize("cross", [False, True])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_dit_block_descriptors_inside_allocations(dt, cross):
    ALLOCS.clear()
    io, host, outs, dev = dit_block_case.build(dt, cross, _HostStorage)
    fields = [n for n, typ in _lib.MiDitBlockIO._fields_ if typ is _lib.MiTensor]
    used = 0
    for name in fields:
        t = getattr(io, name)
        if not t.data:
            assert not cross or not name.startswith("ca_") and name != "norm_ca", name
            continue
        used += 1
        lo, hi = _span(t)
        a = _owner(lo)
        assert a is not None, f"{name}: data pointer outside every allocation"
        assert hi <= a.ptr + a.nbytes, f"{name}: addresses {hi - a.ptr} bytes of a {a.nbytes}-byte allocation"
    assert used == (len(fields) if cross else len(fields) - 9)

    # shape relations the driver's launches rely on
    R = 96 * 2
    for name in ("hidden", "norm_sa", "sa_out", "norm_ffn", "ffn_out") + (("norm_ca", "ca_out") if cross else ()):
        t = getattr(io, name)
        assert t.ne[0] == H and _rows(t) == R, name
    assert io.adaln.ne[0] == 6 * H and io.gate_up.ne[0] == 2 * I and io.ff.ne[0] == I
    assert _rows(io.gate_up) == _rows(io.ff) == R
    assert (io.q.ne[0], io.q.ne[1], io.q.ne[2]) == (D, NH, R) and (io.k.ne[0], io.k.ne[1], io.k.ne[2]) == (D, NKV, R)
    assert io.pos.ne[0] == R and io.q_out.ne[2] == io.k_out.ne[2] == R
    if cross:
        # per-head CA views: [D, S, heads, N] over the projection outputs
        assert (io.ca_q.ne[0], io.ca_q.ne[1], io.ca_q.ne[2]) == (D, 96, NH)
        assert io.ca_q.nb[1] == NH * D * io.ca_q.nb[0] and io.ca_q.nb[2] == D * io.ca_q.nb[0]
        assert (io.ca_k.ne[0], io.ca_k.ne[2]) == (D, NKV)
        assert io.ca_k.nb[1] == 2 * NKV * D * io.ca_k.nb[0]  # the K half of each fused K+V row
        for a, b in (("ca_q", "ca_q_out"), ("ca_k", "ca_k_out")):
            x, y = getattr(io, a), getattr(io, b)
            assert [x.ne[i] for i in range(4)] == [y.ne[i] for i in range(4)]


def test_view_outside_its_allocation_is_refused():
    ALLOCS.clear()
    t = _HostStorage.empty((4, 8), "f32")
    bad = DTensor(t.buf, (4, 9), "f32", (8, 1), 0)  # rows run past the end
    from acestep_ops import ops
    with pytest.raises(ValueError, match="outside"):
        ops.desc(bad)
    ops.desc(t[1:, 2:])


@pytest.mark.parametrize("cross", [False, True])
def test_dit_block_bad_late_operand_returns_before_any_launch(cross):
    """The block's descriptors with the SwiGLU input (the 5th or 7th op of the
    chain) one column short: mi_dit_block_ops reports the shape error (-3)
    rather than the HIP error (-8) the first launch gives on this GPU-less
    host, so nothing ran (and `hidden` was not updated in place)."""
    import ctypes
    ALLOCS.clear()
    io, _, _, _ = dit_block_case.build("bf16", cross, _HostStorage)
    io.gate_up.ne[0] -= 2
    lib = _lib.load()
    assert lib.mi_dit_block_ops(ctypes.byref(io), None) == -3
    io.gate_up.ne[0] += 2
    io.ffn_out.ne[1] -= 1
    assert lib.mi_dit_block_ops(ctypes.byref(io), None) == -3
