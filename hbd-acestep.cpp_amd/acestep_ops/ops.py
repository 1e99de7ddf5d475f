"""Python wrappers over the C ABI, one per ggml op the reference's graph
builders emit (same names, argument meaning and shape rules as the ggml
calls they replace; see include/mi_ops.h for the reference call sites).

Operands are ``device.DTensor`` views: a shape (..., ne1, ne0) maps to the
ggml view [ne0, ne1, ...] with byte strides taken from the element strides.
Q8_0 tensors are uint8 tensors whose last axis holds whole 34-byte blocks
(see ``Q8``). Every call is enqueued on ``stream`` (default: the null
stream); errors raise ``MiError`` with the library's mi_status.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import Q8_0, MiTensor
from .device import DTYPES, DTensor


@dataclass
class Q8:
    """A Q8_0 tensor: ``data`` is a u8 DTensor with shape (..., n_blocks*34)."""
    data: DTensor

    @property
    def ne0(self) -> int:
        return self.data.shape[-1] // 34 * 32

    @property
    def shape(self):
        return tuple(self.data.shape[:-1]) + (self.ne0,)


def desc(t) -> MiTensor:
    """ggml-style descriptor of a DTensor (or Q8) view."""
    d = MiTensor()
    if isinstance(t, Q8):
        x = t.data
        if x.dtype != "u8" or x.shape[-1] % 34 != 0 or x.strides[-1] != 1:
            raise ValueError("Q8 data must be u8 (..., n_blocks*34) with contiguous blocks")
        d.type = Q8_0
        shape = list(t.shape)
        nbytes = [s for s in x.strides]  # u8: element strides are bytes
        nbytes[-1] = 34                  # nb[0] = block size
        blck = 32
    else:
        x = t
        typ = DTYPES[x.dtype][2]
        if typ is None:
            raise TypeError(f"dtype {x.dtype} is not an op operand type")
        d.type = typ
        shape = list(x.shape) or [1]
        nbytes = [s * x.es for s in x.strides] or [x.es]
        blck = 1
    if len(shape) > 4:
        raise ValueError("at most 4 dimensions")
    lo, hi = x.extent()
    if lo < 0 or hi > x.buf.nbytes:
        raise ValueError(f"view bytes [{lo}, {hi}) fall outside its {x.buf.nbytes}-byte allocation")
    ne = shape[::-1]
    nb = nbytes[::-1]
    while len(ne) < 4:  # outer dims of size 1 continue contiguously
        nb.append(nb[-1] * ne[-1] // (blck if len(ne) == 1 else 1))
        ne.append(1)
    d.data = x.ptr
    d.reserved = 0
    for i in range(4):
        d.ne[i] = int(ne[i])
        d.nb[i] = int(nb[i])
    return d


def _p(t):
    return None if t is None else ctypes.byref(desc(t))


def _s(stream):
    return ctypes.c_void_p(stream)


def _out(out, shape, dtype):
    return out if out is not None else DTensor.empty(shape, dtype)


# ---------------------------------------------------------------------------
def rms_norm(x, eps: float, w=None, out=None, stream=None):
    """ggml_rms_norm(x, eps) [* w] over the last axis."""
    y = _out(out, x.shape, x.dtype)
    _lib.call("mi_rms_norm", _p(x), _p(w), eps, _p(y), _s(stream))
    return y


def rms_norm_modulate(x, w, scale, shift, eps: float, out=None, stream=None):
    """((rms_norm(x) * w) * (scale + 1)) + shift  (dit-graph.h:404-405)."""
    y = _out(out, x.shape, x.dtype)
    _lib.call("mi_rms_norm_modulate", _p(x), _p(w), _p(scale), _p(shift), eps, _p(y), _s(stream))
    return y


def add_rms_norm(residual, x, eps: float, gate=None, w=None, scale=None, shift=None, clamp=None, out_sum=None,
                 out_norm=None, stream=None):
    """y_sum = residual + x [* gate] (clamped to `clamp`=(lo, hi) if given);
    y_norm = rms_norm(y_sum) [* w] [* (scale + 1) + shift]. Returns (y_sum, y_norm)."""
    ys = _out(out_sum, residual.shape, residual.dtype)
    yn = _out(out_norm, residual.shape, residual.dtype)
    lo, hi = clamp if clamp is not None else (0.0, 0.0)
    _lib.call("mi_add_rms_norm", _p(residual), _p(x), _p(gate), int(clamp is not None), lo, hi, _p(w), _p(scale),
              _p(shift), eps, _p(ys), _p(yn), _s(stream))
    return ys, yn


def rope_ext(x, pos, n_dims: int, mode: int = 2, freq_base: float = 10000.0, freq_scale: float = 1.0,
             ext_factor: float = 0.0, attn_factor: float = 1.0, out=None, stream=None):
    """ggml_rope_ext. x: (..., n_pos, heads, ne0); pos: i32 (n_pos,)."""
    y = _out(out, x.shape, x.dtype)
    _lib.call("mi_rope_ext", _p(x), _p(pos), n_dims, mode, freq_base, freq_scale, ext_factor, attn_factor, _p(y),
              _s(stream))
    return y


def qk_norm_rope(q, q_w, pos, eps: float, n_dims: int, freq_base: float, k=None, k_w=None, freq_scale=1.0,
                 attn_factor=1.0, q_out=None, k_out=None, stream=None):
    """rope(rms_norm(q) * q_w) and the same for k, in one launch."""
    qo = _out(q_out, q.shape, q.dtype)
    ko = None if k is None else _out(k_out, k.shape, k.dtype)
    _lib.call("mi_qk_norm_rope", _p(q), _p(q_w), _p(qo), _p(k), _p(k_w), _p(ko), _p(pos), eps, n_dims, freq_base,
              freq_scale, attn_factor, _s(stream))
    return qo, ko


def swiglu(gu, swapped: bool = False, out=None, stream=None):
    """ggml_swiglu: gu (..., 2n) -> (..., n)."""
    y = _out(out, gu.shape[:-1] + (gu.shape[-1] // 2,), gu.dtype)
    _lib.call("mi_swiglu", _p(gu), int(bool(swapped)), _p(y), _s(stream))
    return y


def swiglu_split(g, u, out=None, stream=None):
    y = _out(out, g.shape, g.dtype)
    _lib.call("mi_swiglu_split", _p(g), _p(u), _p(y), _s(stream))
    return y


def add(a, b, out=None, stream=None):
    y = _out(out, a.shape, a.dtype)
    _lib.call("mi_add", _p(a), _p(b), _p(y), _s(stream))
    return y


def mul(a, b, out=None, stream=None):
    y = _out(out, a.shape, a.dtype)
    _lib.call("mi_mul", _p(a), _p(b), _p(y), _s(stream))
    return y


def add_clamp(a, b, lo: float = -65504.0, hi: float = 65504.0, out=None, stream=None):
    """ggml_clamp(ggml_add(a, b), lo, hi); b None -> clamp only."""
    y = _out(out, a.shape, a.dtype)
    _lib.call("mi_add_clamp", _p(a), _p(b), lo, hi, _p(y), _s(stream))
    return y


def clamp(x, lo: float, hi: float, out=None, stream=None):
    return add_clamp(x, None, lo, hi, out, stream)


def gated_add(residual, x, gate, out=None, stream=None):
    """residual + x * gate (dit-graph.h:70-76)."""
    y = _out(out, residual.shape, residual.dtype)
    _lib.call("mi_gated_add", _p(residual), _p(x), _p(gate), _p(y), _s(stream))
    return y


def modulate(x, scale, shift, out=None, stream=None):
    """(x * (scale + 1)) + shift (dit-graph.h:54-64)."""
    y = _out(out, x.shape, x.dtype)
    _lib.call("mi_modulate", _p(x), _p(scale), _p(shift), _p(y), _s(stream))
    return y


def get_rows(table, ids, out=None, out_dtype="f32", err=None, stream=None):
    """ggml_get_rows: table (n_rows, n) [or Q8], ids i32 (n_ids,) -> (n_ids, n)."""
    n = table.shape[-1]
    y = _out(out, (ids.shape[0], n), out_dtype)
    ep = ctypes.c_void_p(err.ptr) if err is not None else None
    _lib.call("mi_get_rows", _p(table), _p(ids), _p(y), ep, _s(stream))
    return y


def cpy(src, dst, rounding: int = _lib.Q8_0_CPU_X86, stream=None):
    """ggml_cpy(src, dst) into a same-shape view (Q8 dst quantizes)."""
    _lib.call("mi_cpy_q8_0", _p(src), _p(dst), rounding, _s(stream))
    return dst


def kv_store(k, k_cache, pos0, v=None, v_cache=None, sets=None, rounding: int = _lib.Q8_0_CPU_X86, err=None,
             stream=None):
    """k (B, T, Nkv, D) -> k_cache (n_sets, Nkv, max_seq, D) at slots pos0[b] + t."""
    ep = ctypes.c_void_p(err.ptr) if err is not None else None
    _lib.call("mi_kv_store", _p(k), _p(k_cache), _p(v), _p(v_cache), _p(pos0), _p(sets), rounding, ep, _s(stream))


def qk_norm_rope_kv_store(q, q_w, k, k_w, v, pos, eps: float, n_dims: int, freq_base: float, k_cache, v_cache,
                          pos0, sets=None, clamp_v: bool = False, rounding: int = _lib.Q8_0_CPU_X86, freq_scale=1.0,
                          attn_factor=1.0, q_out=None, err=None, stream=None):
    """qk_norm_rope then kv_store in one launch: q (tokens, Nh, D) -> q_out; k, v (tokens, Nkv, D)
    -> the caches at slots pos0[b] + t (tokens = B sequences x T)."""
    qo = _out(q_out, q.shape, q.dtype)
    ep = ctypes.c_void_p(err.ptr) if err is not None else None
    _lib.call("mi_qk_norm_rope_kv_store", _p(q), _p(q_w), _p(qo), _p(k), _p(k_w), _p(v), _p(pos), eps, n_dims,
              freq_base, freq_scale, attn_factor, int(bool(clamp_v)), _p(k_cache), _p(v_cache), _p(pos0), _p(sets),
              rounding, ep, _s(stream))
    return qo


def scale(x, s: float, out=None, stream=None):
    """ggml_scale: x * s (the timestep scaling in front of the embedding, dit-graph.h:87)."""
    y = _out(out, x.shape, x.dtype)
    _lib.call("mi_scale", _p(x), ctypes.c_float(s), _p(y), _s(stream))
    return y


def timestep_embedding(t, dim: int, max_period: int = 10000, out=None, stream=None):
    y = _out(out, (t.shape[0], dim), "f32")
    _lib.call("mi_timestep_embedding", _p(t), dim, max_period, _p(y), _s(stream))
    return y


def flash_attn_workspace(q, k, v) -> int:
    """Bytes of device workspace mi_flash_attn_ext needs for these operands."""
    n = ctypes.c_size_t(0)
    _lib.call("mi_flash_attn_ext_workspace", _p(q), _p(k), _p(v), ctypes.byref(n))
    return int(n.value)


def flash_attn_ext(q, k, v, mask, scale: float, out=None, workspace=None, max_bias: float = 0.0,
                   logit_softcap: float = 0.0, stream=None):
    """ggml_flash_attn_ext (GGML_PREC_F32). Shapes outermost first:
    q (N, Nh, n_q, D); k, v (Nk3, Nkv, n_kv, D) [or Q8]; mask F16 (mne3, mne2, >= n_q, n_kv) or None;
    returns F32 (N, n_q, Nh, D) -- ggml's [D, Nh, n_q, N]. A workspace of the required size is
    allocated when none is passed."""
    N, Nh, n_q, D = q.shape
    y = _out(out, (N, n_q, Nh, D), "f32")
    need = flash_attn_workspace(q, k, v)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_flash_attn_ext", _p(q), _p(k), _p(v), _p(mask), scale, max_bias, logit_softcap, _p(y), wp, wn,
              _s(stream))
    return y


@dataclass
class Q8R64:
    """A Q8_0 weight [k, n] repacked by mi_q8_0_repack (``data``: u8 DTensor)."""
    data: DTensor
    k: int
    n: int


def q8_0_repack(w, stream=None) -> Q8R64:
    """Load-time repack of a Q8_0 weight ``w`` (Q8, shape (n, k)) for mul_mat_q8_0."""
    n, k = w.shape[-2], w.shape[-1]
    nb = ctypes.c_size_t(0)
    _lib.call("mi_q8_0_repack_bytes", k, n, ctypes.byref(nb))
    dst = DTensor.empty((max(int(nb.value), 1),), "u8")
    _lib.call("mi_q8_0_repack", _p(w), ctypes.c_void_p(dst.ptr), nb.value, _s(stream))
    return Q8R64(dst, k, n)


def mul_mat_q8_0_workspace(w: Q8R64, x) -> int:
    nb = ctypes.c_size_t(0)
    _lib.call("mi_mul_mat_q8_0_workspace", w.k, w.n, _p(x), ctypes.byref(nb))
    return int(nb.value)


def mul_mat_q8_0_noalloc(w: Q8R64, x, out=None, stream=None):
    """mul_mat_q8_0 on the library's static per-GPU scratch: no workspace, no allocation
    in the call (out must then be given by a caller that cannot allocate)."""
    y = _out(out, tuple(x.shape[:-1]) + (w.n,), "f32")
    _lib.call("mi_mul_mat_q8_0_noalloc", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(x), _p(y), _s(stream))
    return y


def mul_mat_q8_0_swiglu_workspace(w: Q8R64, gu) -> int:
    n = ctypes.c_size_t(0)
    _lib.call("mi_mul_mat_q8_0_swiglu_workspace", w.k, w.n, _p(gu), ctypes.byref(n))
    return int(n.value)


def mul_mat_q8_0_swiglu_add(w: Q8R64, gu, r, clamp=None, swapped: bool = False, out=None, workspace=None,
                            stream=None):
    """ggml_add(ggml_mul_mat(w, ggml_swiglu(gu)), r) in one call, then ggml_clamp to
    clamp = (lo, hi) when given: bit-identical to mul_mat_q8_0_swiglu followed by
    add (add_clamp)."""
    y = _out(out, tuple(gu.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_swiglu_workspace(w, gu)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    lo, hi = clamp if clamp is not None else (0.0, 0.0)
    _lib.call("mi_mul_mat_q8_0_swiglu_add", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(gu), int(bool(swapped)), _p(r),
              int(clamp is not None), lo, hi, _p(y), wp, wn, _s(stream))
    return y


def mul_mat_q8_0_swiglu_gated_add(w: Q8R64, gu, r, gate, swapped: bool = False, out=None, workspace=None,
                                  stream=None):
    """r + ggml_mul_mat(w, ggml_swiglu(gu)) * gate in one call (the DiT's gated
    residual after the MLP): bit-identical to mul_mat_q8_0_swiglu followed by gated_add."""
    y = _out(out, tuple(gu.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_swiglu_workspace(w, gu)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_mul_mat_q8_0_swiglu_gated_add", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(gu), int(bool(swapped)),
              _p(r), _p(gate), _p(y), wp, wn, _s(stream))
    return y


def mul_mat_q8_0_swiglu(w: Q8R64, gu, swapped: bool = False, out=None, workspace=None, stream=None):
    """ggml_mul_mat(w, ggml_swiglu(gu)) in one call: gu F32 (m, 2k) -> F32 (m, n),
    bit-identical to swiglu followed by mul_mat_q8_0."""
    y = _out(out, tuple(gu.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_swiglu_workspace(w, gu)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_mul_mat_q8_0_swiglu", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(gu), int(bool(swapped)), _p(y), wp,
              wn, _s(stream))
    return y


def mul_mat_q8_0_rms_norm(w: Q8R64, x, norm_w, eps: float, out=None, workspace=None, stream=None):
    """ggml_mul_mat(w, rms_norm(x) * norm_w) in one call: x F32 (m, k) -> F32 (m, n),
    equal to rms_norm followed by mul_mat_q8_0."""
    y = _out(out, tuple(x.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_workspace(w, x)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_mul_mat_q8_0_rms_norm", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(x), _p(norm_w),
              ctypes.c_float(eps), _p(y), wp, wn, _s(stream))
    return y


def mul_mat_q8_0_add_rms_norm(w: Q8R64, a, b, norm_w, eps: float, out_sum=None, out=None, workspace=None,
                              stream=None):
    """sum = a + b; y = ggml_mul_mat(w, rms_norm(sum) * norm_w) in one call: a, b F32 (m, k)
    -> (sum (m, k), y (m, n)), equal to add_rms_norm followed by mul_mat_q8_0."""
    sm = _out(out_sum, a.shape, "f32")
    y = _out(out, tuple(a.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_workspace(w, a)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_mul_mat_q8_0_add_rms_norm", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(a), _p(b), _p(norm_w),
              ctypes.c_float(eps), _p(sm), _p(y), wp, wn, _s(stream))
    return sm, y


def mul_mat_q8_0_adaln(w: Q8R64, a, norm_w, eps: float, b=None, gate=None, scale=None, shift=None, out_sum=None,
                       out=None, workspace=None, stream=None):
    """The DiT's norm -> product pair in one call (mi_mul_mat_q8_0_adaln): sum = a + b [* gate]
    (with b), x' = rms_norm(sum or a) * norm_w [* (scale + 1) + shift], y = ggml_mul_mat(w, x').
    Returns (sum, y) when b is given, else y; equal to add_rms_norm / rms_norm_modulate
    followed by mul_mat_q8_0."""
    sm = _out(out_sum, a.shape, "f32") if b is not None else None
    y = _out(out, tuple(a.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_workspace(w, a)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_mul_mat_q8_0_adaln", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(a), _p(b), _p(gate), _p(norm_w),
              _p(scale), _p(shift), ctypes.c_float(eps), _p(sm), _p(y), wp, wn, _s(stream))
    return (sm, y) if b is not None else y


def mul_mat_q8_0(w: Q8R64, x, out=None, workspace=None, stream=None):
    """ggml_mul_mat(w, x): x F32 (m, k) with m <= 8 -> F32 (m, n)."""
    y = _out(out, tuple(x.shape[:-1]) + (w.n,), "f32")
    need = mul_mat_q8_0_workspace(w, x)
    ws = workspace
    if need and ws is None:
        ws = DTensor.empty((need,), "u8")
    wp = ctypes.c_void_p(ws.ptr) if ws is not None else None
    wn = ws.numel() * ws.es if ws is not None else 0
    _lib.call("mi_mul_mat_q8_0", ctypes.c_void_p(w.data.ptr), w.k, w.n, _p(x), _p(y), wp, wn, _s(stream))
    return y
