"""The GGUF reader (mi_gguf_*) against files written from the published format
(tests/gguf_writer.py): header, every KV type, tensor infos and data pointers
byte for byte, alignment, and the malformed files the reference's loader
rejects (gguf-weights.h:120-150: a tensor past the end of the file) or that
the format forbids. No GPU: parsing and metadata are host code."""
import ctypes
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "hbd-acestep.cpp_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gguf_writer as gw  # noqa: E402
from acestep_ops import _lib  # noqa: E402
from acestep_ops.gguf import GGUFModel  # noqa: E402
from oracle import oracle as orc  # noqa: E402

L = _lib.load()


def _rng(seed):
    return np.random.default_rng(seed)


def _tensors(seed=0):
    r = _rng(seed)
    f32 = r.standard_normal((3, 5)).astype(np.float32)
    f16 = orc.f32_to_f16(r.standard_normal((2, 4, 8)).astype(np.float32))
    bf16 = orc.f32_to_bf16(r.standard_normal((7,)).astype(np.float32))
    q8 = orc.quantize_q8_0(r.standard_normal((6, 64)).astype(np.float32))
    i32 = r.integers(-9, 9, (2, 3), dtype=np.int32)
    return [("blk.0.attn_q.weight", 0, [5, 3], f32), ("blk.0.ffn.weight", 1, [8, 4, 2], f16),
            ("norm.weight", 30, [7], bf16), ("token_embd.weight", 8, [64, 6], q8), ("pos", 26, [3, 2], i32)]


def _write(tmp_path, kv, tensors, name="m.gguf", **kw):
    data, start = gw.build(kv, [(n, t, ne, gw.tensor_bytes(a)) for n, t, ne, a in tensors], **kw)
    p = tmp_path / name
    p.write_bytes(data)
    return str(p), start


KV = [("general.architecture", gw.STR, "acestep-dit"), ("acestep-dit.block_count", gw.U32, 24),
      ("acestep-dit.rope.freq_base", gw.F32, 1e4), ("acestep.flag", gw.BOOL, True), ("a.u8", gw.U8, 200),
      ("a.i8", gw.I8, -5), ("a.u16", gw.U16, 60000), ("a.i16", gw.I16, -300), ("a.i32", gw.I32, -70000),
      ("a.u64", gw.U64, 2 ** 40 + 3), ("a.i64", gw.I64, -(2 ** 40)), ("a.f64", gw.F64, 0.125),
      ("a.arr", gw.ARR, (gw.U32, [1, 2, 3])), ("a.strs", gw.ARR, (gw.STR, ["x", "yz", ""])),
      ("a.empty", gw.STR, "")]


@pytest.mark.parametrize("alignment,version", [(None, 3), (64, 3), (32, 2)])
def test_round_trip(tmp_path, alignment, version):
    ts = _tensors(1)
    path, start = _write(tmp_path, KV, ts, alignment=alignment, version=version)
    with GGUFModel(path) as g:
        assert g.n_tensors == len(ts)
        assert g.tensor_names() == [t[0] for t in ts]
        for name, typ, ne, arr in ts:
            t = g.tensor_info(name)
            assert t.type == typ and t.n_dims == len(ne)
            assert [t.ne[d] for d in range(4)] == ne + [1] * (4 - len(ne))
            assert t.nbytes == arr.nbytes
            assert ctypes.string_at(t.data, t.nbytes) == arr.tobytes()
        assert g.tensor_info("missing") is None
        assert g.get_u32("acestep-dit.block_count") == 24
        assert g.get_f32("acestep-dit.rope.freq_base") == np.float32(1e4)
        assert g.get_bool("acestep.flag") is True
        assert g.get_str("general.architecture") == "acestep-dit"
        assert g.get_str("a.empty") == ""
        # absent keys read as the reference's getters read them
        assert g.get_u32("nope") == 0 and g.get_f32("nope") == 0.0 and g.get_str("nope") == ""
        assert g.get_bool("nope") is False
        keys = dict(g.keys())
        assert keys["a.arr"] == gw.ARR and keys["a.u64"] == gw.U64 and keys["a.strs"] == gw.ARR
        assert ("general.alignment" in keys) == (alignment is not None)
        # a typed getter on another type is an error, not a reinterpretation
        with pytest.raises(_lib.MiError):
            g.get_u32("a.i32")
        with pytest.raises(_lib.MiError):
            g.get_f32("a.f64")


def test_data_section_alignment(tmp_path):
    """Tensor data starts at the header end rounded up to general.alignment and each
    tensor at its offset from there."""
    ts = _tensors(2)
    for al in (32, 128, 256):
        path, start = _write(tmp_path, KV[:2], ts, name=f"a{al}.gguf", alignment=al)
        assert start % al == 0
        raw = open(path, "rb").read()
        with GGUFModel(path) as g:
            for name, _, _, arr in ts:
                t = g.tensor_info(name)
                mv = ctypes.string_at(t.data, t.nbytes)
                i = raw.find(arr.tobytes(), start)
                assert mv == raw[i:i + t.nbytes] and (i - start) % al == 0


def _rc(path):
    h = ctypes.c_void_p()
    rc = L.mi_gguf_open(path.encode(), ctypes.byref(h))
    if rc == 0:
        L.mi_gguf_close(h)
    return rc


def test_malformed_files(tmp_path):
    ts = _tensors(3)
    tb = [(n, t, ne, gw.tensor_bytes(a)) for n, t, ne, a in ts]
    good, _ = gw.build(KV, tb)

    def put(name, data):
        p = tmp_path / name
        p.write_bytes(data)
        return str(p)

    assert _rc(put("good.gguf", good)) == 0
    assert _rc(str(tmp_path / "absent.gguf")) == -9
    assert _rc(put("trunc.gguf", good[:-40])) == -9                      # last tensor runs past the end
    assert _rc(put("trunc_head.gguf", good[:50])) == -9
    assert _rc(put("magic.gguf", b"GGUX" + good[4:])) == -9
    assert _rc(put("v1.gguf", gw.build(KV, tb, version=1)[0])) == -9
    assert _rc(put("misaligned.gguf", gw.build(KV, tb, offsets=[0, 8, 64, 96, 200])[0])) == -9
    assert _rc(put("dup.gguf", gw.build(KV, tb + [tb[0]])[0])) == -9     # duplicate tensor name
    assert _rc(put("dupkey.gguf", gw.build(KV + [KV[1]], tb)[0])) == -9
    assert _rc(put("al3.gguf", gw.build(KV, tb, alignment=3)[0])) == -9  # alignment not a power of two
    assert _rc(put("qrow.gguf", gw.build(KV, [("q", 8, [48, 2], b"\0" * 102)])[0])) == -9  # ne0 % 32
    assert _rc(put("type.gguf", gw.build(KV, [("x", 99, [4], b"\0" * 16)])[0])) == -2      # unknown ggml type
    bad_kv = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw._str("k") + struct.pack("<II", 77, 0)  # unknown KV type
    assert _rc(put("kvtype.gguf", bad_kv)) == -9
    nested = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw._str("n") + struct.pack("<IIQ", gw.ARR, gw.ARR, 1)
    assert _rc(put("nested.gguf", nested + struct.pack("<IQ", gw.U8, 0))) == -9
    # element or byte counts that overflow 64 bits (a wrapped product would describe
    # a huge tensor over a 0-byte region)
    assert _rc(put("nel_ovf.gguf", gw.build(KV, [("x", 0, [2 ** 61, 2 ** 61, 16], b"")])[0])) == -9
    assert _rc(put("nb_ovf.gguf", gw.build(KV, [("x", 0, [2 ** 60, 2], b"")])[0])) == -9
    assert _rc(put("q8_ovf.gguf", gw.build(KV, [("x", 8, [2 ** 61, 2 ** 2], b"")])[0])) == -9
    huge = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 60)
    assert _rc(put("hugestr.gguf", huge)) == -9


def test_null_arguments():
    h = ctypes.c_void_p()
    assert L.mi_gguf_open(None, ctypes.byref(h)) == -1
    assert L.mi_gguf_n_tensors(None) == -1
    assert L.mi_gguf_find_tensor(None, b"x") == -1
    L.mi_gguf_close(None)


def test_mutated_files_never_read_outside(tmp_path):
    """Seeded byte flips, overwritten lengths and truncations of a valid file: each
    open either fails with a status or yields tensors whose bytes lie inside the
    mapping (every byte is read back here)."""
    ts = _tensors(4)
    good, _ = gw.build(KV, [(n, t, ne, gw.tensor_bytes(a)) for n, t, ne, a in ts])
    r = _rng(5)
    p = tmp_path / "mut.gguf"
    opened = 0
    for it in range(400):
        b = bytearray(good)
        kind = it % 4
        if kind == 0:
            for _ in range(r.integers(1, 6)):
                b[r.integers(0, len(b))] = r.integers(0, 256)
        elif kind == 1:
            i = r.integers(0, len(b) - 8)
            b[i:i + 8] = struct.pack("<Q", int(r.integers(0, 1 << 62)))
        elif kind == 2:
            b = b[:r.integers(0, len(b))]
        else:
            i = r.integers(24, 400)
            b[i:i + 4] = struct.pack("<I", int(r.integers(0, 1 << 32)))
        p.write_bytes(bytes(b))
        h = ctypes.c_void_p()
        rc = L.mi_gguf_open(str(p).encode(), ctypes.byref(h))
        assert rc in (0, -9, -2), rc
        if rc == 0:
            opened += 1
            t = _lib.MiGGUFTensor()
            for i in range(L.mi_gguf_n_tensors(h)):
                assert L.mi_gguf_get_tensor(h, i, ctypes.byref(t)) == 0
                ctypes.string_at(t.data, t.nbytes)
            L.mi_gguf_close(h)
    assert opened > 0
