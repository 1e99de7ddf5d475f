"""Minimal device-memory plumbing over the HIP runtime that libmi_ops.so links.

libmi_ops.so is compiled by this image's ROCm toolchain and links that
ROCm's libamdhip64; device buffers, copies, streams and events here go
through the very same runtime instance (it is resolved by soname after the
library is loaded), so the library never runs under a different, older HIP
runtime than the one its code objects were built for.

Host<->device copies are staged through buffers allocated with hipHostMalloc:
a copy from pageable memory makes the runtime lock the caller's existing
pages, which some deployments refuse.

``DTensor`` is a strided view (shape / element strides / byte offset) over a
``Buffer``; it supports the few view operations the tests and the benchmark
need (basic slicing, view/reshape of contiguous data, unflatten, permute).
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _lib

_hip = None

# dtype name -> (element size, numpy storage dtype, mi_type)
DTYPES = {
    "f32": (4, np.float32, _lib.F32),
    "bf16": (2, np.uint16, _lib.BF16),
    "f16": (2, np.uint16, _lib.F16),
    "i32": (4, np.int32, _lib.I32),
    "u8": (1, np.uint8, None),
}

H2D, D2H, D2D = 1, 2, 3


class HipError(RuntimeError):
    pass


def hip():
    """ctypes handle of the HIP runtime libmi_ops.so is linked against."""
    global _hip
    if _hip is None:
        _lib.load()  # pulls in its libamdhip64 first; the soname then resolves to it
        h = ctypes.CDLL("libamdhip64.so.7")
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        sig = {
            "hipMalloc": [ctypes.POINTER(vp), sz],
            "hipFree": [vp],
            "hipHostMalloc": [ctypes.POINTER(vp), sz, ctypes.c_uint],
            "hipHostFree": [vp],
            "hipMemcpy": [vp, vp, sz, i],
            "hipMemcpyAsync": [vp, vp, sz, i, vp],
            "hipMemset": [vp, i, sz],
            "hipMemsetAsync": [vp, i, sz, vp],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [vp],
            "hipStreamCreate": [ctypes.POINTER(vp)],
            "hipStreamDestroy": [vp],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipGetDeviceCount": [ctypes.POINTER(i)],
            "hipSetDevice": [i],
            "hipGetLastError": [],
            "hipRuntimeGetVersion": [ctypes.POINTER(i)],
            "hipDeviceGetAttribute": [ctypes.POINTER(i), i, i],
            "hipStreamBeginCapture": [vp, i],
            "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, sz],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
        }
        for name, args in sig.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        h.hipGetErrorString.argtypes = [ctypes.c_int]
        h.hipGetErrorString.restype = ctypes.c_char_p
        _hip = h
    return _hip


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise HipError(f"{what}: {hip().hipGetErrorString(rc).decode()} ({rc})")


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = hip().hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def runtime_version() -> int:
    v = ctypes.c_int(0)
    check(hip().hipRuntimeGetVersion(ctypes.byref(v)), "hipRuntimeGetVersion")
    return v.value


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Buffer:
    """One hipMalloc allocation; freed when the last view is dropped."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    def __del__(self):
        if getattr(self, "ptr", None) and _hip is not None:
            _hip.hipFree(self.ptr)
            self.ptr = None


class PinnedBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(hip().hipHostMalloc(ctypes.byref(p), max(self.nbytes, 1), 0), "hipHostMalloc")
        self.ptr = p.value

    def array(self, dtype, count):
        return np.frombuffer((ctypes.c_char * self.nbytes).from_address(self.ptr), dtype=dtype, count=count)

    def __del__(self):
        if getattr(self, "ptr", None) and _hip is not None:
            _hip.hipHostFree(self.ptr)
            self.ptr = None


def _contig_strides(shape):
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= d
    return tuple(reversed(st))


class DTensor:
    """Strided view of device memory (element strides, byte offset)."""

    def __init__(self, buf: Buffer, shape, dtype: str, strides=None, offset: int = 0):
        assert dtype in DTYPES, dtype
        self.buf = buf
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.strides = tuple(strides) if strides is not None else _contig_strides(self.shape)
        self.offset = int(offset)

    # ---- construction --------------------------------------------------
    @staticmethod
    def empty(shape, dtype="f32"):
        shape = tuple(shape) if isinstance(shape, (tuple, list)) else (shape,)
        return DTensor(Buffer(math.prod(shape) * DTYPES[dtype][0]), shape, dtype)

    @staticmethod
    def zeros(shape, dtype="f32"):
        t = DTensor.empty(shape, dtype)
        t.fill_byte(0)
        return t

    @staticmethod
    def full_byte(shape, value: int, dtype="u8"):
        t = DTensor.empty(shape, dtype)
        t.fill_byte(value)
        return t

    @staticmethod
    def from_numpy(a: np.ndarray, dtype: str | None = None):
        """Upload a host array (for bf16/f16 pass uint16 bit patterns with dtype='bf16'/'f16')."""
        if dtype is None:
            dtype = {np.dtype(np.float32): "f32", np.dtype(np.int32): "i32", np.dtype(np.uint8): "u8"}[a.dtype]
        es, npdt, _ = DTYPES[dtype]
        a = np.ascontiguousarray(a).view(npdt) if a.dtype != npdt else np.ascontiguousarray(a)
        t = DTensor.empty(a.shape, dtype)
        if a.nbytes:
            stage = PinnedBuffer(a.nbytes)
            ctypes.memmove(stage.ptr, a.ctypes.data, a.nbytes)
            check(hip().hipMemcpy(t.ptr, stage.ptr, a.nbytes, H2D), "hipMemcpy H2D")
        return t

    # ---- properties ----------------------------------------------------
    @property
    def es(self) -> int:
        return DTYPES[self.dtype][0]

    @property
    def ptr(self) -> int:
        return self.buf.ptr + self.offset

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def numel(self) -> int:
        return math.prod(self.shape)

    def extent(self):
        """Byte range [lo, hi) of the buffer this view can address (lo == hi when empty)."""
        if self.numel() == 0:
            return self.offset, self.offset
        lo = hi = self.offset
        for n, s in zip(self.shape, self.strides):
            if s >= 0:
                hi += (n - 1) * s * self.es
            else:
                lo += (n - 1) * s * self.es
        return lo, hi + self.es

    def is_contiguous(self) -> bool:
        return self.strides == _contig_strides(self.shape)

    def fill_byte(self, value: int) -> None:
        assert self.is_contiguous()
        check(hip().hipMemset(self.ptr, int(value), self.numel() * self.es), "hipMemset")

    # ---- views ---------------------------------------------------------
    def __getitem__(self, idx):
        if not isinstance(idx, tuple):
            idx = (idx,)
        shape, strides, off = [], [], self.offset
        d = 0
        for it in idx:
            if it is Ellipsis:
                rest = self.ndim - d - (len(idx) - idx.index(Ellipsis) - 1)
                for _ in range(rest):
                    shape.append(self.shape[d])
                    strides.append(self.strides[d])
                    d += 1
                continue
            if isinstance(it, int):
                i = it if it >= 0 else it + self.shape[d]
                assert 0 <= i < self.shape[d]
                off += i * self.strides[d] * self.es
                d += 1
                continue
            start, stop, step = it.indices(self.shape[d])
            assert step > 0
            n = max(0, (stop - start + step - 1) // step)
            off += start * self.strides[d] * self.es
            shape.append(n)
            strides.append(self.strides[d] * step)
            d += 1
        while d < self.ndim:
            shape.append(self.shape[d])
            strides.append(self.strides[d])
            d += 1
        return DTensor(self.buf, shape, self.dtype, strides, off)

    def view(self, *shape):
        shape = shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape
        shape = list(shape)
        if -1 in shape:
            k = shape.index(-1)
            shape[k] = self.numel() // max(1, math.prod(s for s in shape if s != -1))
        assert math.prod(shape) == self.numel() and self.is_contiguous(), "view needs contiguous data"
        return DTensor(self.buf, shape, self.dtype, None, self.offset)

    reshape = view

    def unflatten(self, dim: int, sizes):
        dim = dim % self.ndim
        assert math.prod(sizes) == self.shape[dim]
        inner = _contig_strides(sizes)
        shape = self.shape[:dim] + tuple(sizes) + self.shape[dim + 1:]
        strides = self.strides[:dim] + tuple(s * self.strides[dim] for s in inner) + self.strides[dim + 1:]
        return DTensor(self.buf, shape, self.dtype, strides, self.offset)

    def permute(self, *dims):
        return DTensor(self.buf, [self.shape[d] for d in dims], self.dtype, [self.strides[d] for d in dims],
                       self.offset)

    def reinterpret(self, dtype: str):
        """Same bytes, another element type of equal size (e.g. u16 bits as bf16)."""
        assert DTYPES[dtype][0] == self.es
        return DTensor(self.buf, self.shape, dtype, self.strides, self.offset)

    # ---- host copies ---------------------------------------------------
    def numpy(self) -> np.ndarray:
        """Download (bf16/f16 come back as uint16 bit patterns)."""
        es, npdt, _ = DTYPES[self.dtype]
        if not self.is_contiguous():
            # gather the view through a contiguous device copy made by the host
            full = DTensor(self.buf, (self.buf.nbytes // es,), self.dtype, None, 0).numpy()
            base = self.offset // es
            idx = np.zeros(self.shape, np.int64) + base
            for d, (n, s) in enumerate(zip(self.shape, self.strides)):
                sh = [1] * self.ndim
                sh[d] = n
                idx = idx + (np.arange(n, dtype=np.int64) * s).reshape(sh)
            return full[idx]
        n = self.numel() * es
        out = np.empty(self.shape, npdt)
        if n:
            stage = PinnedBuffer(n)
            check(hip().hipMemcpy(stage.ptr, self.ptr, n, D2H), "hipMemcpy D2H")
            ctypes.memmove(out.ctypes.data, stage.ptr, n)
        return out

    def item(self):
        return self.numpy().reshape(-1)[0].item()


class Stream:
    """A HIP stream at the default priority."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(hip().hipStreamCreate(ctypes.byref(h)), "hipStreamCreate")
        self.handle = h.value

    def synchronize(self):
        check(hip().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def __del__(self):
        if getattr(self, "handle", None) and _hip is not None:
            _hip.hipStreamDestroy(self.handle)
            self.handle = None


class Graph:
    """Stream-captured HIP graph: ``with g.capture(stream): <launches>``, then ``g.launch()``."""

    RELAXED = 2  # hipStreamCaptureModeRelaxed

    def __init__(self):
        self.graph = None
        self.exec = None
        self.stream = None

    def capture(self, stream: "Stream"):
        g = self

        class _Ctx:
            def __enter__(self):
                g.stream = stream
                check(hip().hipStreamBeginCapture(stream.handle, Graph.RELAXED), "hipStreamBeginCapture")
                return g

            def __exit__(self, et, ev, tb):
                graph = ctypes.c_void_p()
                rc = hip().hipStreamEndCapture(stream.handle, ctypes.byref(graph))
                if et is None:
                    check(rc, "hipStreamEndCapture")
                    g.graph = graph.value
                    ex = ctypes.c_void_p()
                    check(hip().hipGraphInstantiate(ctypes.byref(ex), g.graph, None, None, 0), "hipGraphInstantiate")
                    g.exec = ex.value
                return False

        return _Ctx()

    def launch(self):
        check(hip().hipGraphLaunch(self.exec, self.stream.handle), "hipGraphLaunch")

    def __del__(self):
        if _hip is not None:
            if getattr(self, "exec", None):
                _hip.hipGraphExecDestroy(self.exec)
            if getattr(self, "graph", None):
                _hip.hipGraphDestroy(self.graph)


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.h = e.value

    def record(self, stream=None):
        check(hip().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self):
        check(hip().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        if getattr(self, "h", None) and _hip is not None:
            _hip.hipEventDestroy(self.h)
            self.h = None
