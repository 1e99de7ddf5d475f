"""CPU oracle for the per-layer fused ops -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``oracle/_build/liborc.so`` (plain-C restatement of the
ggml-cpu arithmetic, ``oracle/ggml_cpu_ref.c``). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg may import
this module, and only as the parity reference or the timed CPU baseline.

Each primitive below is one ggml graph node. The chain functions at the end
call them in the order the reference's graph builders emit them, citing the
builder lines, so a fused GPU kernel is compared against the unfused ggml
node sequence it replaces.

bf16 activations (measured beside the reference's F32; the reference computes in F32) are
checked as: bf16 -> f32 (exact), the fp32 node chain, f32 -> bf16 (RNE).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liborc.so")
_lib = None

F32, F16, Q8_0, I32, BF16 = 0, 1, 8, 26, 30
QK8_0, Q8_0_SIZE = 32, 34

_fp = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def build() -> str:
    """Compile the oracle library (make in oracle/)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def use_isa(isa: str) -> str:
    """Load the x86-64-v3 build ("v3", the one the tests use) or the x86-64-v4 build
    ("v4", AVX-512) of the same source; only before the first call into it."""
    global _LIB_PATH
    path = os.path.join(_HERE, "_build", "liborc.so" if isa == "v3" else f"liborc_{isa}.so")
    if _lib is not None and path != _LIB_PATH:
        raise RuntimeError("the oracle library is already loaded")
    _LIB_PATH = path
    return path


class Rock4(ctypes.Structure):
    """orc_rock4: ROCK4 tables (degrees, finishing and recurrence coefficients)."""
    _fields_ = [("ms", _i32p), ("fpa", ctypes.POINTER(ctypes.c_double)), ("fpb", ctypes.POINTER(ctypes.c_double)),
                ("recf", ctypes.POINTER(ctypes.c_double)), ("ms_len", ctypes.c_int), ("recf_len", ctypes.c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_rms_norm_f32.argtypes = [_fp, _i64, _i64, ctypes.c_float, _fp]
        L.orc_add_f32.argtypes = [_fp, _fp, _i64, _i64, _i64, _i64, _fp]
        L.orc_mul_f32.argtypes = [_fp, _fp, _i64, _i64, _i64, _i64, _fp]
        L.orc_clamp_f32.argtypes = [_fp, _i64, ctypes.c_float, ctypes.c_float, _fp]
        L.orc_scale_f32.argtypes = [_fp, _i64, ctypes.c_float, _fp]
        L.orc_rope_neox_f32.argtypes = [_fp, _i64, _i64, _i64, ctypes.c_int, _i32p, ctypes.c_float,
                                        ctypes.c_float, ctypes.c_float, _fp]
        L.orc_rope_theta_scale.argtypes = [ctypes.c_float, ctypes.c_int]
        L.orc_rope_theta_scale.restype = ctypes.c_float
        L.orc_swiglu_f32.argtypes = [_fp, _i64, _fp, _i64, _i64, _i64, _fp]
        L.orc_quantize_rows_q8_0.argtypes = [_fp, _i64, _i64, ctypes.c_int, _u8p]
        L.orc_dequantize_row_q8_0.argtypes = [_u8p, _fp, _i64]
        L.orc_get_rows.argtypes = [ctypes.c_void_p, ctypes.c_int, _i64, _i64, _i32p, _i64, _fp]
        L.orc_get_rows.restype = ctypes.c_int
        L.orc_timestep_embedding_f32.argtypes = [_fp, _i64, ctypes.c_int, ctypes.c_int, _fp]
        L.orc_fp32_to_fp16_n.argtypes = [_fp, _u16p, _i64]
        L.orc_fp16_to_fp32_n.argtypes = [_u16p, _fp, _i64]
        L.orc_fp32_to_bf16_n.argtypes = [_fp, _u16p, _i64]
        L.orc_bf16_to_fp32_n.argtypes = [_u16p, _fp, _i64]
        L.orc_flash_attn_ext.argtypes = [_fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                         ctypes.c_float, ctypes.c_int, _fp]
        L.orc_flash_attn_ext_f16acc.argtypes = [_fp, _fp, _u16p, _fp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                _i64, ctypes.c_float, ctypes.c_int, _fp, _fp]
        L.orc_mul_mat_q8_0.argtypes = [_u8p, _fp, _i64, _i64, _i64, _fp]
        _dp = ctypes.POINTER(ctypes.c_double)
        L.orc_apg_forward.argtypes = [_fp, _fp, _i64, _i64, _i64, ctypes.c_float, ctypes.c_double, ctypes.c_float,
                                      _dp, ctypes.c_int, _fp]
        L.orc_flow_step.argtypes = [ctypes.c_int, _fp, _fp, _i64, ctypes.c_float, ctypes.c_float, ctypes.c_int, _fp,
                                    _fp]
        L.orc_flow_final.argtypes = [_fp, _fp, _i64, ctypes.c_float, _fp]
        L.orc_sde_step.argtypes = [_fp, _fp, _fp, _i64, ctypes.c_float, ctypes.c_float]
        L.orc_stork4_step.argtypes = [_fp, _fp, _i64, ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                      ctypes.c_float, _fp, _fp, ctypes.c_int, ctypes.POINTER(Rock4), _i32p]
        L.orc_dcw.argtypes = [ctypes.c_int, _fp, _fp, _i64, _i64, _i64, ctypes.c_float, ctypes.c_float,
                              ctypes.c_float, ctypes.c_float]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_get_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------------------
# number formats
# ---------------------------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = _c32(x)
    y = np.empty(x.shape, np.uint16)
    lib().orc_fp32_to_bf16_n(_f(x), y.ctypes.data_as(_u16p), x.size)
    return y


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_fp32_n(h.ctypes.data_as(_u16p), _f(y), h.size)
    return y


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = _c32(x)
    y = np.empty(x.shape, np.uint16)
    lib().orc_fp32_to_fp16_n(_f(x), y.ctypes.data_as(_u16p), x.size)
    return y


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_fp16_to_fp32_n(h.ctypes.data_as(_u16p), _f(y), h.size)
    return y


# ---------------------------------------------------------------------------
# primitives: one ggml node each. Arrays are numpy, innermost axis = ggml ne0.
# ---------------------------------------------------------------------------
def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    """ggml_rms_norm over the last axis."""
    x = _c32(x)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().orc_rms_norm_f32(_f(x), x.size // n, n, eps, _f(y))
    return y


def _bin(fn, a, b):
    a = _c32(a)
    b = _c32(b)
    n = a.shape[-1]
    bn = b.shape[-1]
    rows = a.size // n
    brows = b.size // bn
    assert n % bn == 0 and rows % brows == 0, "b must repeat into a (ggml_can_repeat)"
    y = np.empty_like(a)
    fn(_f(a), _f(b), rows, n, brows, bn, _f(y))
    return y


def add(a, b) -> np.ndarray:
    """ggml_add (b broadcast by repetition)."""
    return _bin(lib().orc_add_f32, a, b)


def mul(a, b) -> np.ndarray:
    """ggml_mul (b broadcast by repetition)."""
    return _bin(lib().orc_mul_f32, a, b)


def clamp(x, lo: float, hi: float) -> np.ndarray:
    """ggml_clamp."""
    x = _c32(x)
    y = np.empty_like(x)
    lib().orc_clamp_f32(_f(x), x.size, lo, hi, _f(y))
    return y


def scale(x, s: float) -> np.ndarray:
    """ggml_scale."""
    x = _c32(x)
    y = np.empty_like(x)
    lib().orc_scale_f32(_f(x), x.size, s, _f(y))
    return y


def rope_theta_scale(freq_base: float, n_dims: int) -> float:
    return float(lib().orc_rope_theta_scale(freq_base, n_dims))


def rope_neox(x, pos, n_dims: int, freq_base: float, freq_scale: float = 1.0, attn_factor: float = 1.0):
    """ggml_rope_ext mode NEOX. x: (..., n_pos, heads, ne0); positions index the
    n_pos axis (ggml ne2); leading axes (ggml ne3) reuse the same positions."""
    x = _c32(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    n_pos, heads, ne0 = x.shape[-3:]
    assert pos.shape == (n_pos,)
    outer = x.size // (n_pos * heads * ne0)
    y = np.empty_like(x)
    xs = x.reshape(outer, n_pos * heads * ne0)
    ys = y.reshape(outer, n_pos * heads * ne0)
    for o in range(outer):
        xo = np.ascontiguousarray(xs[o])
        yo = np.empty_like(xo)
        lib().orc_rope_neox_f32(_f(xo), n_pos, heads, ne0, n_dims, pos.ctypes.data_as(_i32p), freq_base,
                                freq_scale, attn_factor, _f(yo))
        ys[o] = yo
    return y


def swiglu_split(g, u) -> np.ndarray:
    """ggml_swiglu_split(g, u)."""
    g = _c32(g)
    u = _c32(u)
    assert g.shape == u.shape
    n = g.shape[-1]
    rows = g.size // n
    y = np.empty_like(g)
    lib().orc_swiglu_f32(_f(g), n, _f(u), n, rows, n, _f(y))
    return y


def swiglu(gu, swapped: bool = False) -> np.ndarray:
    """ggml_swiglu(gu): gate = first half of ne0 (second half when swapped)."""
    gu = _c32(gu)
    n2 = gu.shape[-1]
    assert n2 % 2 == 0
    n = n2 // 2
    g, u = (gu[..., n:], gu[..., :n]) if swapped else (gu[..., :n], gu[..., n:])
    return swiglu_split(g, u)


def quantize_q8_0(x, variant: str = "x86") -> np.ndarray:
    """Rows of x (last axis, multiple of 32) -> Q8_0 bytes, shape (..., n/32*34).
    variant "ref" = quantize_row_q8_0_ref; "x86" = ggml-cpu x86 from_float."""
    x = _c32(x)
    n = x.shape[-1]
    assert n % QK8_0 == 0
    rows = x.size // n
    y = np.empty(x.shape[:-1] + (n // QK8_0 * Q8_0_SIZE,), np.uint8)
    lib().orc_quantize_rows_q8_0(_f(x), rows, n, 0 if variant == "ref" else 1, y.ctypes.data_as(_u8p))
    return y


def dequantize_q8_0(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rb = q.shape[-1]
    assert rb % Q8_0_SIZE == 0
    n = rb // Q8_0_SIZE * QK8_0
    rows = q.size // rb
    y = np.empty(q.shape[:-1] + (n,), np.float32)
    lib().orc_dequantize_row_q8_0(q.ctypes.data_as(_u8p), _f(y), rows * n)
    return y


def get_rows(table: np.ndarray, type_: int, n: int, ids) -> np.ndarray:
    """ggml_get_rows: table rows (raw bytes or typed array) gathered by ids -> F32."""
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    row_bytes = {F32: 4 * n, F16: 2 * n, BF16: 2 * n, Q8_0: n // QK8_0 * Q8_0_SIZE}[type_]
    n_rows = table.nbytes // row_bytes
    y = np.zeros(ids.shape + (n,), np.float32)
    rc = lib().orc_get_rows(table.ctypes.data, type_, n_rows, n, ids.ctypes.data_as(_i32p), ids.size, _f(y))
    if rc != 0:
        raise IndexError("get_rows: id out of range")
    return y


def timestep_embedding(t, dim: int, max_period: int = 10000) -> np.ndarray:
    """ggml_timestep_embedding: t[n] -> (n, dim)."""
    t = _c32(t).reshape(-1)
    y = np.empty((t.size, dim), np.float32)
    lib().orc_timestep_embedding_f32(_f(t), t.size, dim, max_period, _f(y))
    return y


QCONV = {"f32": 0, "f16": 1, "bf16": 2, "q8_0": 3}


def flash_attn_ext(q, k, v, mask, scale: float, k_type: str = "f16") -> np.ndarray:
    """ggml_flash_attn_ext (max_bias 0, softcap 0), exact value in double.
    q (N, Nh, n_q, D); k, v (N, Nkv, n_kv, D) as F32 values (dequantized);
    mask (mN, mH, mQ, n_kv) F32 values of the F16 mask, or None.
    k_type names K's storage type: q is converted as ggml-cpu converts it.
    Returns (N, n_q, Nh, D), ggml's [D, Nh, n_q, N] result."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    N, Nh, n_q, D = q.shape
    _, Nkv, n_kv, _ = k.shape
    assert k.shape == v.shape == (N, Nkv, n_kv, D) and Nh % Nkv == 0 and D <= 1024
    if mask is not None:
        mask = _c32(mask)
        mN, mH, mQ, mk = mask.shape
        assert mk == n_kv and mQ >= n_q
        mp = _f(mask)
    else:
        mN = mH = mQ = 1
        mp = None
    y = np.empty((N, n_q, Nh, D), np.float32)
    lib().orc_flash_attn_ext(_f(q), _f(k), _f(v), mp, N, Nh, Nkv, n_q, n_kv, D, mN, mH, mQ, scale, QCONV[k_type],
                             _f(y))
    return y


def flash_attn_ext_f16acc(q, k, v16, mask, scale: float, k_type: str = "f16"):
    """ggml-cpu's flash attention for an F16 V: the output accumulated in fp16
    one key at a time (see orc_flash_attn_ext_f16acc). v16: uint16 fp16 bits
    (N, Nkv, n_kv, D); other arguments as flash_attn_ext. Returns (y, bud):
    y (N, n_q, Nh, D) and, per element, the fp16 accumulation's rounding
    errors carried to y."""
    q, k = _c32(q), _c32(k)
    v16 = np.ascontiguousarray(v16, dtype=np.uint16)
    N, Nh, n_q, D = q.shape
    _, Nkv, n_kv, _ = k.shape
    assert k.shape == v16.shape == (N, Nkv, n_kv, D) and Nh % Nkv == 0 and D <= 1024
    if mask is not None:
        mask = _c32(mask)
        mN, mH, mQ, mk = mask.shape
        assert mk == n_kv and mQ >= n_q
        mp = _f(mask)
    else:
        mN = mH = mQ = 1
        mp = None
    y = np.empty((N, n_q, Nh, D), np.float32)
    bud = np.empty((N, n_q, Nh, D), np.float32)
    lib().orc_flash_attn_ext_f16acc(_f(q), _f(k), v16.ctypes.data_as(_u16p), mp, N, Nh, Nkv, n_q, n_kv, D, mN, mH,
                                    mQ, scale, QCONV[k_type], _f(y), _f(bud))
    return y, bud


# ---------------------------------------------------------------------------
# chains: unfused ggml node sequences that each fused kernel replaces
# ---------------------------------------------------------------------------
def rms_norm_mul(x, w, eps):
    """qwen3_rms_norm (qwen3-enc.h:114-120) / dit_ggml_rms_norm_weighted
    (dit-graph.h:24-30): ggml_mul(ggml_rms_norm(x, eps), w)."""
    return mul(rms_norm(x, eps), w)


def adaln_modulate(norm, scale_v, shift_v):
    """dit_ggml_adaln (dit-graph.h:54-64): (norm * (scale + 1)) + shift, with
    one_plus_s = ggml_add(scale, one[1]) computed on the [H] vector first."""
    one_plus_s = add(scale_v, np.ones(1, np.float32))
    return add(mul(norm, one_plus_s), shift_v)


def rms_norm_modulate(x, w, scale_v, shift_v, eps):
    """DiT pre-attention / pre-FFN chain (dit-graph.h:404-405, 442-443)."""
    return adaln_modulate(rms_norm_mul(x, w, eps), scale_v, shift_v)


def gated_add(residual, x, gate):
    """dit_ggml_gated_add (dit-graph.h:70-76): residual + (x * gate)."""
    return add(residual, mul(x, gate))


def add_clamp(a, b, lo=-65504.0, hi=65504.0):
    """Residual add + FP16 clamp (qwen3-lm.h:479-482, 730-733)."""
    return clamp(add(a, b), lo, hi)


def qk_norm_rope(x, w, pos, eps, n_dims, freq_base, freq_scale=1.0, attn_factor=1.0):
    """QK-norm then NEOX rope (qwen3-lm.h:372-379, 660-667; qwen3-enc.h:165-174;
    dit-graph.h:183-196): rope(mul(rms_norm(x), w)). x: (..., n_pos, heads, D).
    w None -> plain rope (no norm)."""
    y = x if w is None else rms_norm_mul(x, w, eps)
    return rope_neox(y, pos, n_dims, freq_base, freq_scale, attn_factor)


def bf16_chain(fn, *arrays_bf16, out_bf16=True, **kw):
    """Run an fp32 chain on bf16 inputs (bf16 -> f32 exact), round the output to bf16."""
    xs = [bf16_to_f32(a) if isinstance(a, np.ndarray) and a.dtype == np.uint16 else a for a in arrays_bf16]
    y = fn(*xs, **kw)
    return f32_to_bf16(y) if out_bf16 else y


def mul_mat_q8_0(w: np.ndarray, x) -> np.ndarray:
    """ggml_mul_mat(w, x): w Q8_0 bytes (n, k/32*34), x F32 (m, k) -> F32 (m, n)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = _c32(x)
    n = w.shape[0]
    k = w.shape[1] // Q8_0_SIZE * QK8_0
    assert x.shape[-1] == k
    m = x.size // k if k else 0
    y = np.empty((m, n), np.float32)
    lib().orc_mul_mat_q8_0(w.ctypes.data_as(_u8p), _f(x), n, k, m, _f(y))
    return y


def apg_forward(cond, uncond, scale: float, ra: np.ndarray, first: bool, momentum: float = -0.75,
                threshold: float = 2.5) -> np.ndarray:
    """APG over samples: cond, uncond F32 (n, t, oc); ra float64 (n, t, oc), updated in place."""
    cond, uncond = _c32(cond), _c32(uncond)
    assert ra.dtype == np.float64 and ra.flags.c_contiguous and ra.shape == cond.shape
    n, t, oc = cond.shape
    out = np.empty_like(cond)
    lib().orc_apg_forward(_f(cond), _f(uncond), n, t, oc, scale, momentum, threshold,
                          ra.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), int(first), _f(out))
    return out


SOLVERS = {"euler": 0, "dpm3m": 1}


def flow_step(solver: str, xt: np.ndarray, vt, t_curr: float, t_next: float, hist: int = 0, prev=None,
              prev2=None) -> None:
    """One solver step, in place on xt (and prev/prev2 for dpm3m); all F32 contiguous."""
    vt = _c32(vt)
    assert xt.dtype == np.float32 and xt.flags.c_contiguous
    z = np.zeros(1, np.float32)
    pp = prev if prev is not None else z
    p2 = prev2 if prev2 is not None else z
    lib().orc_flow_step(SOLVERS[solver], _f(xt), _f(vt), xt.size, t_curr, t_next, hist, _f(pp), _f(p2))


def flow_final(xt, vt, t: float) -> np.ndarray:
    xt, vt = _c32(xt), _c32(vt)
    out = np.empty_like(xt)
    lib().orc_flow_final(_f(xt), _f(vt), xt.size, t, _f(out))
    return out


def sde_step(xt: np.ndarray, vt, noise, t_curr: float, t_next: float) -> None:
    """SDE ancestral step in place on xt (solver-sde.h:33-36) with the given N(0,1) draws."""
    vt, noise = _c32(vt), _c32(noise)
    assert xt.dtype == np.float32 and xt.flags.c_contiguous and vt.size == xt.size == noise.size
    lib().orc_sde_step(_f(xt), _f(vt), _f(noise), xt.size, t_curr, t_next)


def rock4_struct(ms, fpa, fpb, recf):
    """Keep-alive tuple (Rock4, arrays) for ROCK4 tables given as numpy arrays."""
    ms = np.ascontiguousarray(ms, np.int32)
    fpa = np.ascontiguousarray(fpa, np.float64).reshape(len(ms), 6)
    fpb = np.ascontiguousarray(fpb, np.float64).reshape(len(ms), 4)
    recf = np.ascontiguousarray(recf, np.float64)
    dp = ctypes.POINTER(ctypes.c_double)
    r = Rock4(ms.ctypes.data_as(_i32p), fpa.ctypes.data_as(dp), fpb.ctypes.data_as(dp), recf.ctypes.data_as(dp),
              len(ms), len(recf))
    return r, (ms, fpa, fpb, recf)


def stork4_step(xt: np.ndarray, vt, t_curr: float, t_next: float, hist: int, h1: float, h2: float,
                prev: np.ndarray, prev2: np.ndarray, substeps: int, tables) -> tuple:
    """STORK4 step in place on xt, prev, prev2 (solver-stork.h:269-323); tables = (ms, fpa, fpb, recf).
    Returns (derivative order, accepted degree or 0, Euler fallback)."""
    vt = _c32(vt)
    for a in (xt, prev, prev2):
        assert a.dtype == np.float32 and a.flags.c_contiguous and a.size == vt.size
    r, keep = rock4_struct(*tables)
    info = np.zeros(3, np.int32)
    lib().orc_stork4_step(_f(xt), _f(vt), xt.size, t_curr, t_next, hist, h1, h2, _f(prev), _f(prev2), substeps,
                          ctypes.byref(r), info.ctypes.data_as(_i32p))
    del keep
    return int(info[0]), int(info[1]), bool(info[2])


DCW_MODES = {"low": 0, "high": 1, "double": 2, "pix": 3}


def dcw(mode: str, xt: np.ndarray, vt, t_curr: float, t_next: float, scaler: float, high_scaler: float = 0.0) -> None:
    """DCW correction in place on xt (n, t, oc) after a solver step (dit-sampler.h:626-664)."""
    vt = _c32(vt)
    assert xt.dtype == np.float32 and xt.flags.c_contiguous and xt.ndim == 3 and vt.shape == xt.shape
    n, t, oc = xt.shape
    lib().orc_dcw(DCW_MODES.get(mode, 0), _f(xt), _f(vt), n, t, oc, t_curr, t_next, scaler, high_scaler)
