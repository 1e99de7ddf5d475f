"""A minimal GGUF writer for tests, written from the published GGUF format
(versions 2/3, little-endian): magic "GGUF", u32 version, u64 tensor count,
u64 KV count; KV = string key, u32 value type, value; tensor info = string
name, u32 n_dims, u64 ne[n_dims] (ggml order), u32 ggml type, u64 offset into
the data section; the data section starts at the header end rounded up to
general.alignment (default 32), and every tensor offset is a multiple of it.
Strings are u64 length + bytes; arrays are u32 element type, u64 count,
elements. Test infrastructure: it produces files for the reader under test.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _val(t, v) -> bytes:
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for x in items:
            out += _val(et, x)
        return out
    return struct.pack(_FMT[t], v)


def build(kv, tensors, alignment=None, version=3, offsets=None, magic=b"GGUF", pad_data=True):
    """kv: [(key, type, value)]; tensors: [(name, ggml_type, ne (ggml order), bytes)].
    Returns the file bytes. `offsets` overrides the tensor offsets (for malformed files)."""
    kv = list(kv)
    if alignment is not None:
        kv.append(("general.alignment", U32, alignment))
    al = alignment or 32
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, t, v in kv:
        head += _str(k) + struct.pack("<I", t) + _val(t, v)
    offs, at = [], 0
    for _, _, _, data in tensors:
        offs.append(at)
        at += (len(data) + al - 1) // al * al
    if offsets is not None:
        offs = offsets
    for (name, typ, ne, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", typ, off)
    data_start = (len(head) + al - 1) // al * al
    out = bytearray(head + b"\0" * (data_start - len(head)))
    for (_, _, _, data), off in zip(tensors, offs):
        end = data_start + off + len(data)
        if len(out) < end:
            out += b"\0" * (end - len(out))
        out[data_start + off:end] = data
    if pad_data and tensors:
        out += b"\0" * ((-len(out)) % al)
    return bytes(out), data_start


def tensor_bytes(a: np.ndarray) -> bytes:
    return np.ascontiguousarray(a).tobytes()
