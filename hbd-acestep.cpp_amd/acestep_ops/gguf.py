"""GGUF weights through the library's reader (mi_gguf_*), with the reference
loader's names and behaviour (gguf-weights.h): GGUFModel.load = gf_load,
load_tensor = gf_load_tensor, load_tensor_f32 = gf_load_tensor_f32,
load_qkv_fused = gf_load_qkv_fused, load_pair_fused = gf_load_pair_fused,
get_u32 / get_f32 / get_str / get_bool = gf_get_* (0 / 0.0 / "" / False when
the key is absent). Tensors come back as device DTensors; shapes are given
outermost first, as DTensor shapes are (ggml ne reversed)."""
from __future__ import annotations

import ctypes

from . import _lib
from ._lib import MiError, MiGGUFTensor
from .device import DTensor

# ggml type -> DTensor dtype for the types the ops take; Q8_0 comes back as a Q8
_DT = {0: "f32", 1: "f16", 30: "bf16", 26: "i32"}
Q8_0 = 8


class GGUFModel:
    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _lib.call("mi_gguf_open", str(path).encode(), ctypes.byref(h))
        self._h = h

    @classmethod
    def load(cls, path: str) -> "GGUFModel":
        return cls(path)

    def close(self) -> None:
        if self._h:
            _lib.load().mi_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- metadata ----------------------------------------------------------
    @property
    def n_tensors(self) -> int:
        return int(_lib.load().mi_gguf_n_tensors(self._h))

    def keys(self):
        L = _lib.load()
        out = []
        for i in range(int(L.mi_gguf_n_kv(self._h))):
            k, t = ctypes.c_char_p(), ctypes.c_int32()
            _lib.call("mi_gguf_get_key", self._h, i, ctypes.byref(k), ctypes.byref(t))
            out.append((k.value.decode(), int(t.value)))
        return out

    def _get(self, fn, key, ctype, default):
        v = ctype()
        rc = getattr(_lib.load(), fn)(self._h, key.encode(), ctypes.byref(v))
        if rc == -6:  # absent
            return default
        if rc != 0:
            raise MiError(fn, rc)
        return v.value

    def get_u32(self, key: str) -> int:
        return int(self._get("mi_gguf_get_u32", key, ctypes.c_uint32, 0))

    def get_f32(self, key: str) -> float:
        return float(self._get("mi_gguf_get_f32", key, ctypes.c_float, 0.0))

    def get_bool(self, key: str) -> bool:
        return bool(self._get("mi_gguf_get_bool", key, ctypes.c_int, 0))

    def get_str(self, key: str) -> str:
        v = self._get("mi_gguf_get_str", key, ctypes.c_char_p, b"")
        return v.decode() if isinstance(v, bytes) else v

    def tensor_info(self, name: str) -> MiGGUFTensor | None:
        i = int(_lib.load().mi_gguf_find_tensor(self._h, name.encode()))
        if i < 0:
            return None
        t = MiGGUFTensor()
        _lib.call("mi_gguf_get_tensor", self._h, i, ctypes.byref(t))
        return t

    def tensor_names(self):
        out = []
        for i in range(self.n_tensors):
            t = MiGGUFTensor()
            _lib.call("mi_gguf_get_tensor", self._h, i, ctypes.byref(t))
            out.append(t.name.decode())
        return out

    # -- device tensors ----------------------------------------------------
    @staticmethod
    def _shape(t: MiGGUFTensor):
        return tuple(int(t.ne[d]) for d in range(t.n_dims))[::-1]

    def _alloc(self, t: MiGGUFTensor, ne1: int | None = None):
        shape = list(self._shape(t))
        if ne1 is not None:
            shape = [ne1] + shape[1:] if len(shape) == 2 else [ne1, shape[-1]]
        if t.type == Q8_0:
            from .ops import Q8
            blocks = shape[-1] // 32
            return Q8(DTensor.empty(tuple(shape[:-1]) + (blocks * 34,), "u8"))
        if t.type not in _DT:
            raise MiError("gguf tensor type", -2)
        return DTensor.empty(tuple(shape), _DT[t.type])

    @staticmethod
    def _ptr_bytes(d):
        x = d.data if hasattr(d, "data") and isinstance(getattr(d, "data"), DTensor) else d
        return x.ptr, x.numel() * x.es

    def load_tensor(self, name: str):
        t = self.tensor_info(name)
        if t is None:
            raise KeyError(f"tensor '{name}' not found")
        d = self._alloc(t)
        p, n = self._ptr_bytes(d)
        _lib.call("mi_gguf_upload", self._h, name.encode(), 0, ctypes.c_void_p(p), n, None)
        return d

    def try_load_tensor(self, name: str):
        return None if self.tensor_info(name) is None else self.load_tensor(name)

    def load_tensor_f32(self, name: str):
        t = self.tensor_info(name)
        if t is None:
            raise KeyError(f"tensor '{name}' not found")
        if t.type not in (0, 1, 30):
            return self.load_tensor(name)  # the reference loads other types as they are
        d = DTensor.empty(self._shape(t), "f32")
        _lib.call("mi_gguf_upload", self._h, name.encode(), 1, ctypes.c_void_p(d.ptr), d.numel() * 4, None)
        return d

    def _fused(self, names):
        ts = [self.tensor_info(n) for n in names]
        if any(t is None for t in ts):
            raise KeyError(f"tensor not found among {names}")
        if any(t.type != ts[0].type for t in ts):
            return None  # the caller loads them separately
        ne1 = sum(int(t.ne[1]) for t in ts)
        d = self._alloc(ts[0], ne1)
        p, n = self._ptr_bytes(d)
        arr = (ctypes.c_char_p * len(names))(*[x.encode() for x in names])
        out = ctypes.c_int64()
        _lib.call("mi_gguf_upload_rows", self._h, arr, len(names), ctypes.c_void_p(p), n, ctypes.byref(out), None)
        return d

    def load_qkv_fused(self, q: str, k: str, v: str):
        return self._fused([q, k, v])

    def load_pair_fused(self, a: str, b: str):
        return self._fused([a, b])
