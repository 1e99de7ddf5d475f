"""CPU-only checks of the C-ABI library: it loads, exports every entry point
declared in include/mi_ops.h, and rejects invalid descriptors with the right
mi_status before any launch (so these calls never touch a GPU)."""
import ctypes
import os
import re

import pytest

from helpers import ROOT

from acestep_ops import _lib
from acestep_ops._lib import BF16, F32, I32, Q8_0, MiTensor

HEADER = os.path.join(ROOT, "include", "mi_ops.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|int64_t|void|const char \*)\s+(mi_\w+)\s*\(", src, flags=re.M)))


def test_library_loads_and_exports_header_symbols():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), f"{name} not exported"
    assert set(names) == set(_lib.PROTOTYPES), "ctypes prototypes out of sync with mi_ops.h"
    assert lib.mi_abi_version() == 2
    assert lib.mi_status_str(-3) == b"inconsistent shapes"


def _t(shape, typ=F32, data=4096, nb=None):
    """Descriptor with a fake (never dereferenced) data pointer."""
    es = {F32: 4, I32: 4, BF16: 2, 1: 2, Q8_0: 34}[typ]
    ne = list(shape) + [1] * (4 - len(shape))
    d = MiTensor()
    d.data = data
    d.type = typ
    d.reserved = 0
    if nb is None:
        nb = [es]
        row = es * ne[0] // (32 if typ == Q8_0 else 1)
        nb += [row, row * ne[1], row * ne[1] * ne[2]]
    for i in range(4):
        d.ne[i] = ne[i]
        d.nb[i] = nb[i]
    return d


R = ctypes.byref
L = _lib.load()
NULL_S = None


def test_rms_norm_validation():
    x, y, w = _t([1024, 8]), _t([1024, 8]), _t([1024])
    assert L.mi_rms_norm(None, None, 1e-6, R(y), NULL_S) == -1
    assert L.mi_rms_norm(R(x), None, 1e-6, R(_t([1024, 9])), NULL_S) == -3
    assert L.mi_rms_norm(R(x), R(_t([512])), 1e-6, R(y), NULL_S) == -3
    assert L.mi_rms_norm(R(x), R(_t([1024], BF16)), 1e-6, R(y), NULL_S) == -2
    assert L.mi_rms_norm(R(_t([1024, 8], I32)), None, 1e-6, R(y), NULL_S) == -2
    assert L.mi_rms_norm(R(x), R(w), -1.0, R(y), NULL_S) == -6
    assert L.mi_rms_norm(R(x), R(w), float("nan"), R(y), NULL_S) == -6
    bad_inner = _t([1024, 8], nb=[8, 8192, 65536, 65536])
    assert L.mi_rms_norm(R(bad_inner), None, 1e-6, R(y), NULL_S) == -4
    assert L.mi_rms_norm(R(_t([1024, 8], data=4098)), None, 1e-6, R(y), NULL_S) == -5
    null_data = _t([1024, 8], data=0)
    assert L.mi_rms_norm(R(null_data), None, 1e-6, R(y), NULL_S) == -1
    reserved = _t([1024, 8])
    reserved.reserved = 1
    assert L.mi_rms_norm(R(reserved), None, 1e-6, R(y), NULL_S) == -6
    assert L.mi_rms_norm_modulate(R(x), None, R(w), R(w), 1e-6, R(y), NULL_S) == -1
    assert L.mi_rms_norm_modulate(R(x), R(w), R(_t([1023])), R(w), 1e-6, R(y), NULL_S) == -3


def test_add_rms_norm_validation():
    a, x, ys, yn, w = _t([2048, 8]), _t([2048, 8], data=8192), _t([2048, 8], data=16384), _t([2048, 8], data=32768), _t([2048])
    f = L.mi_add_rms_norm
    assert f(R(a), R(x), None, 0, 0.0, 0.0, R(w), None, None, 1e-6, R(ys), R(_t([2048, 9])), NULL_S) == -3
    assert f(R(a), R(_t([2048, 8], BF16)), None, 0, 0.0, 0.0, R(w), None, None, 1e-6, R(ys), R(yn), NULL_S) == -2
    assert f(R(a), R(x), R(_t([2047])), 0, 0.0, 0.0, R(w), None, None, 1e-6, R(ys), R(yn), NULL_S) == -3
    assert f(R(a), R(x), None, 0, 0.0, 0.0, None, R(w), R(w), 1e-6, R(ys), R(yn), NULL_S) == -1    # modulate needs w
    assert f(R(a), R(x), None, 0, 0.0, 0.0, R(w), R(w), None, 1e-6, R(ys), R(yn), NULL_S) == -1    # scale without shift
    assert f(R(a), R(x), None, 1, float("nan"), 1.0, R(w), None, None, 1e-6, R(ys), R(yn), NULL_S) == -6
    assert f(R(a), R(x), None, 0, 0.0, 0.0, R(w), None, None, 1e-6, R(ys), R(a), NULL_S) == -6     # y_norm aliases


def test_rope_validation():
    x, y = _t([128, 16, 32]), _t([128, 16, 32])
    pos = _t([32], I32)
    assert L.mi_rope_ext(R(x), R(pos), 128, 0, 1e4, 1.0, 0.0, 1.0, R(y), NULL_S) == -7   # NORMAL mode
    assert L.mi_rope_ext(R(x), R(pos), 128, 2, 1e4, 1.0, 1.0, 1.0, R(y), NULL_S) == -7   # YaRN ext_factor
    assert L.mi_rope_ext(R(x), R(_t([31], I32)), 128, 2, 1e4, 1.0, 0.0, 1.0, R(y), NULL_S) == -3
    assert L.mi_rope_ext(R(x), R(_t([32])), 128, 2, 1e4, 1.0, 0.0, 1.0, R(y), NULL_S) == -2
    assert L.mi_rope_ext(R(x), R(pos), 127, 2, 1e4, 1.0, 0.0, 1.0, R(y), NULL_S) == -6
    assert L.mi_rope_ext(R(x), R(pos), 256, 2, 1e4, 1.0, 0.0, 1.0, R(y), NULL_S) == -6
    assert L.mi_rope_ext(R(x), R(pos), 128, 2, -1.0, 1.0, 0.0, 1.0, R(y), NULL_S) == -6
    k = _t([128, 8, 32])
    w = _t([128])
    assert L.mi_qk_norm_rope(R(x), R(w), R(y), R(k), None, R(k), R(pos), 1e-6, 128, 1e6, 1.0, 1.0, NULL_S) == -6
    assert L.mi_qk_norm_rope(R(x), R(w), R(y), R(k), R(w), None, R(pos), 1e-6, 128, 1e6, 1.0, 1.0, NULL_S) == -1
    assert L.mi_qk_norm_rope(R(x), R(w), R(y), R(_t([64, 8, 32])), R(w), R(_t([64, 8, 32])), R(pos), 1e-6, 128,
                             1e6, 1.0, 1.0, NULL_S) == -3
    kb = _t([128, 8, 32], BF16)
    assert L.mi_qk_norm_rope(R(x), R(w), R(y), R(kb), R(w), R(kb), R(pos), 1e-6, 128, 1e6, 1.0, 1.0, NULL_S) == -2


def test_swiglu_and_binary_validation():
    gu, y = _t([6144, 4]), _t([3072, 4])
    assert L.mi_swiglu(R(_t([6143, 4])), 0, R(y), NULL_S) == -3
    assert L.mi_swiglu(R(gu), 0, R(_t([3072, 5])), NULL_S) == -3
    # rows not uniformly strided (nb2 != ne1*nb1)
    odd = _t([6144, 4, 2], nb=[4, 24576, 24576 * 5, 24576 * 10])
    assert L.mi_swiglu(R(odd), 0, R(_t([3072, 4, 2])), NULL_S) == -4
    assert L.mi_swiglu_split(R(_t([64, 2])), R(_t([64, 2], BF16)), R(_t([64, 2])), NULL_S) == -2
    a = _t([2048, 8])
    assert L.mi_add(R(a), None, R(a), NULL_S) == -1
    assert L.mi_add(R(a), R(_t([2048, 3])), R(a), NULL_S) == -3      # cannot repeat 3 into 8
    assert L.mi_gated_add(R(a), R(a), R(_t([2048], BF16)), R(a), NULL_S) == -2
    assert L.mi_modulate(R(a), R(_t([2047])), R(_t([2048])), R(a), NULL_S) == -3
    assert L.mi_add_clamp(R(a), R(a), float("nan"), 1.0, R(a), NULL_S) == -6


def test_q8_get_rows_kv_validation():
    tab = _t([1024, 100], Q8_0)
    ids = _t([16], I32)
    y = _t([1024, 16])
    assert L.mi_get_rows(R(_t([1000, 100], Q8_0)), R(ids), R(y), None, NULL_S) == -3   # ne0 % 32
    assert L.mi_get_rows(R(tab), R(_t([16])), R(y), None, NULL_S) == -2
    assert L.mi_get_rows(R(tab), R(ids), R(_t([1024, 15])), None, NULL_S) == -3
    assert L.mi_get_rows(R(tab), R(ids), R(_t([1024, 16], I32)), None, NULL_S) == -2
    assert L.mi_get_rows(R(tab), R(ids), R(y), ctypes.c_void_p(4098), NULL_S) == -5
    assert L.mi_get_rows(R(_t([1024, 100, 2], Q8_0)), R(ids), R(y), None, NULL_S) == -7
    src, dst = _t([128, 8, 4]), _t([128, 8, 4], Q8_0)
    assert L.mi_cpy_q8_0(R(src), R(dst), 5, NULL_S) == -6
    assert L.mi_cpy(R(src), R(_t([128, 8, 5], Q8_0)), NULL_S) == -3
    assert L.mi_cpy(R(_t([128, 8, 4], Q8_0)), R(dst), NULL_S) == -2
    k = _t([128, 8, 16, 4])
    cache = _t([128, 1024, 8, 4], Q8_0)
    pos0 = _t([4], I32)
    assert L.mi_kv_store(R(k), R(cache), None, None, R(_t([3], I32)), None, 0, None, NULL_S) == -3
    assert L.mi_kv_store(R(k), R(_t([128, 1024, 4, 4], Q8_0)), None, None, R(pos0), None, 0, None, NULL_S) == -3
    assert L.mi_kv_store(R(k), R(cache), R(k), None, R(pos0), None, 0, None, NULL_S) == -1
    assert L.mi_kv_store(R(k), R(cache), None, None, R(pos0), R(_t([4])), 0, None, NULL_S) == -2
    assert L.mi_kv_store(R(k), R(cache), R(k), R(_t([128, 1024, 8, 4], BF16)), R(pos0), None, 0, None,
                         NULL_S) == -3
    assert L.mi_timestep_embedding(R(_t([4])), 0, 10000, R(_t([0, 4])), NULL_S) == -6
    assert L.mi_timestep_embedding(R(_t([4])), 256, 10000, R(_t([256, 5])), NULL_S) == -3


def test_qk_norm_rope_kv_store_validation():
    D, Nh, Nkv, n_tok = 128, 32, 8, 8
    q, qo = _t([D, Nh, n_tok], BF16), _t([D, Nh, n_tok], BF16)
    k, v = _t([D, Nkv, n_tok], BF16), _t([D, Nkv, n_tok], BF16)
    w, pos, pos0 = _t([D]), _t([n_tok], I32), _t([8], I32)
    kc, vc = _t([D, 512, Nkv, 8], Q8_0), _t([D, 512, Nkv, 8], Q8_0)
    f = L.mi_qk_norm_rope_kv_store

    def call(q=q, qw=w, qo=qo, k=k, kw=w, v=v, pos=pos, n_dims=D, kc=kc, vc=vc, pos0=pos0, sets=None, rounding=0,
             err=None):
        return f(R(q) if q else None, R(qw) if qw else None, R(qo) if qo else None, R(k) if k else None,
                 R(kw) if kw else None, R(v) if v else None, R(pos) if pos else None, 1e-6, n_dims, 1e6, 1.0, 1.0, 0,
                 R(kc) if kc else None, R(vc) if vc else None, R(pos0) if pos0 else None, R(sets) if sets else None,
                 rounding, err, NULL_S)

    assert call(v=None) == -1
    assert call(kc=None) == -1
    assert call(kw=None) == -6                                   # one norm weight without the other
    assert call(v=_t([D, Nkv, n_tok + 1], BF16)) == -3
    assert call(v=_t([D, Nkv, n_tok])) == -2                      # V of another type
    assert call(qo=_t([D, Nh, n_tok])) == -2                      # q_out of another type
    assert call(pos=_t([n_tok + 1], I32)) == -3
    assert call(n_dims=3) == -6
    assert call(vc=_t([D, 512, Nkv, 8], 1)) == -3                 # caches of different types
    assert call(kc=_t([D, 512, Nkv + 1, 8], Q8_0), vc=_t([D, 512, Nkv + 1, 8], Q8_0)) == -3
    assert call(pos0=_t([3], I32)) == -3                          # 8 tokens are not 3 sequences
    assert call(sets=_t([8])) == -2
    assert call(rounding=5) == -6
    assert call(err=ctypes.c_void_p(4098)) == -5
    assert call(n_dims=64) == -7                                  # partial rotation: the three calls


def test_flash_attn_validation():
    D, n_q, Nh, N, n_kv, Nkv = 128, 1, 32, 8, 256, 8
    q = _t([D, n_q, Nh, N])
    k = _t([D, n_kv, Nkv, N], 1)     # F16
    v = _t([D, n_kv, Nkv, N], 1)
    y = _t([D, Nh, n_q, N])
    mask = _t([n_kv, 1, 1, N], 1)
    ws = ctypes.c_size_t(0)
    fa = L.mi_flash_attn_ext
    assert fa(R(q), R(k), R(v), R(mask), 0.1, 0.0, 0.0, None, None, 0, NULL_S) == -1
    assert fa(R(q), R(k), R(v), R(mask), 0.1, 0.5, 0.0, R(y), None, 0, NULL_S) == -7      # max_bias (ALiBi)
    assert fa(R(q), R(k), R(v), R(mask), 0.1, 0.0, 30.0, R(y), None, 0, NULL_S) == -7     # logit softcap
    assert fa(R(q), R(k), R(v), R(mask), float("nan"), 0.0, 0.0, R(y), None, 0, NULL_S) == -6
    assert fa(R(q), R(k), R(_t([D, n_kv, Nkv, N], Q8_0)), R(mask), 0.1, 0.0, 0.0, R(y), None, 0, NULL_S) == -2
    assert fa(R(_t([D, n_q, Nh, N], I32)), R(k), R(v), R(mask), 0.1, 0.0, 0.0, R(y), None, 0, NULL_S) == -2
    assert fa(R(q), R(k), R(v), R(mask), 0.1, 0.0, 0.0, R(_t([D, Nh, n_q, N], BF16)), None, 0, NULL_S) == -2
    assert fa(R(q), R(_t([D, n_kv, 5, N], 1)), R(_t([D, n_kv, 5, N], 1)), None, 0.1, 0.0, 0.0, R(y), None, 0,
              NULL_S) == -3                                                                 # Nh % Nkv
    assert fa(R(q), R(k), R(v), R(_t([n_kv + 1, 1, 1, N], 1)), 0.1, 0.0, 0.0, R(y), None, 0, NULL_S) == -3
    assert fa(R(q), R(k), R(v), R(_t([n_kv, 1, 1, N])), 0.1, 0.0, 0.0, R(y), None, 0, NULL_S) == -2  # F32 mask
    assert fa(R(q), R(k), R(v), R(mask), 0.1, 0.0, 0.0, R(_t([D, Nh, n_q + 1, N])), None, 0, NULL_S) == -3
    q96, k96 = _t([96, n_q, Nh, N]), _t([96, n_kv, Nkv, N], 1)
    assert fa(R(q96), R(k96), R(k96), None, 0.1, 0.0, 0.0, R(_t([96, Nh, n_q, N])), None, 0, NULL_S) == -7
    kodd = _t([D, n_kv, Nkv, N], 1, nb=[2, 264, 264 * n_kv, 264 * n_kv * Nkv])  # rows 8-byte aligned only
    assert fa(R(q), R(kodd), R(kodd), None, 0.1, 0.0, 0.0, R(y), None, 0, NULL_S) == -5
    # a split key range needs the workspace the query reports
    assert L.mi_flash_attn_ext_workspace(R(q), R(k), R(v), ctypes.byref(ws)) == 0
    big = _t([D, 8192, Nkv, N], Q8_0)
    assert L.mi_flash_attn_ext_workspace(R(q), R(big), R(big), ctypes.byref(ws)) == 0 and ws.value > 0
    assert fa(R(q), R(big), R(big), None, 0.1, 0.0, 0.0, R(y), None, 0, NULL_S) == -6
    assert fa(R(q), R(big), R(big), None, 0.1, 0.0, 0.0, R(y), ctypes.c_void_p(4096), ws.value - 1, NULL_S) == -6
    assert L.mi_flash_attn_ext_workspace(R(q), R(k), R(v), None) == -1
    for qs in ([64, 1, 2, 0], [64, 0, 2, 1], [64, 1, 2, 1]):  # empty batch, no queries, no keys
        k0 = _t([64, 0, 2, 1], 1)
        assert L.mi_flash_attn_ext_workspace(R(_t(qs)), R(k0), R(k0), ctypes.byref(ws)) == 0 and ws.value == 0


def test_mul_mat_q8_0_validation():
    k, n, m = 256, 100, 8
    x = _t([k, m])
    y = _t([n, m])
    nb = ctypes.c_size_t(0)
    mm = L.mi_mul_mat_q8_0
    W = ctypes.c_void_p(4096)
    assert L.mi_q8_0_repack_bytes(k, n, ctypes.byref(nb)) == 0 and nb.value == 2 * (k // 32) * 2176
    assert L.mi_q8_0_repack_bytes(k + 16, n, ctypes.byref(nb)) == -3        # k % 32
    assert L.mi_q8_0_repack_bytes(k, n, None) == -1
    assert L.mi_q8_0_repack(R(_t([k, n])), W, 1 << 20, NULL_S) == -2          # F32 weight
    assert L.mi_q8_0_repack(R(_t([k, n], Q8_0)), W, 10, NULL_S) == -6         # dst too small
    assert mm(W, k, n, R(x), None, None, 0, NULL_S) == -1
    assert mm(W, k, n, R(_t([k, 9])), R(_t([n, 9])), None, 0, NULL_S) == -6   # long x: the matrix kernel, no workspace
    assert mm(W, k, n, R(_t([k + 32, m])), R(y), None, 0, NULL_S) == -3
    assert mm(W, k, n, R(x), R(_t([n + 1, m])), None, 0, NULL_S) == -3
    assert mm(W, k, n, R(_t([k, m], BF16)), R(y), None, 0, NULL_S) == -2
    assert mm(W, k, n, R(x), R(_t([n, m], BF16)), None, 0, NULL_S) == -2
    assert mm(ctypes.c_void_p(4098), k, n, R(x), R(y), None, 0, NULL_S) == -5  # weight alignment
    assert L.mi_mul_mat_q8_0_workspace(k, n, R(x), ctypes.byref(nb)) == 0 and nb.value > 0
    assert mm(W, k, n, R(x), R(y), None, 0, NULL_S) == -6                     # no workspace
    assert mm(W, k, n, R(x), R(y), ctypes.c_void_p(1 << 20), nb.value - 1, NULL_S) == -6
    assert mm(W, k, n, R(x), R(y), ctypes.c_void_p((1 << 20) + 16), nb.value, NULL_S) == -5
    assert L.mi_mul_mat_q8_0_workspace(k, n, R(_t([k, 0])), ctypes.byref(nb)) == 0 and nb.value == 0
    assert L.mi_mul_mat_q8_0_workspace(k, 0, R(x), ctypes.byref(nb)) == 0 and nb.value == 0
    # the allocation-free variant: same checks, and a scratch need above the static array
    na = L.mi_mul_mat_q8_0_noalloc
    assert na(W, k, n, R(x), None, NULL_S) == -1
    assert na(W, k, n, R(_t([k + 32, m])), R(y), NULL_S) == -3
    assert na(ctypes.c_void_p(4098), k, n, R(x), R(y), NULL_S) == -5
    big_k, big_m = 8192, 8192                                                 # 64 MiB of quantized x
    assert L.mi_mul_mat_q8_0_workspace(big_k, 64, R(_t([big_k, big_m])), ctypes.byref(nb)) == 0
    assert nb.value > _lib.NOALLOC_SCRATCH_BYTES
    assert na(W, big_k, 64, R(_t([big_k, big_m])), R(_t([64, big_m])), NULL_S) == -10
    assert L.mi_status_str(-10) == b"needs more scratch than the library's static buffer holds"
    # the norm prologue: norm_w F32 [k]
    mn = L.mi_mul_mat_q8_0_rms_norm
    nw = _t([k])
    assert L.mi_mul_mat_q8_0_workspace(k, n, R(x), ctypes.byref(nb)) == 0
    assert mn(W, k, n, R(x), None, ctypes.c_float(1e-6), R(y), None, 0, NULL_S) == -1
    assert mn(W, k, n, R(x), R(_t([k], BF16)), ctypes.c_float(1e-6), R(y), None, 0, NULL_S) == -2
    assert mn(W, k, n, R(x), R(_t([k + 32])), ctypes.c_float(1e-6), R(y), None, 0, NULL_S) == -3
    assert mn(W, k, n, R(x), R(nw), ctypes.c_float(-1.0), R(y), None, 0, NULL_S) == -6
    assert mn(W, k, n, R(x), R(nw), ctypes.c_float(1e-6), R(y), None, 0, NULL_S) == -6   # no workspace
    assert mn(W, k, n, R(x), R(nw), ctypes.c_float(1e-6), None, None, 0, NULL_S) == -1
    # with the residual add: sum = a + b must not overlap a or b
    ma = L.mi_mul_mat_q8_0_add_rms_norm
    eps = ctypes.c_float(1e-6)
    assert ma(W, k, n, R(x), None, R(nw), eps, R(x), R(y), None, 0, NULL_S) == -1
    assert ma(W, k, n, R(x), R(_t([k, m])), R(nw), eps, None, R(y), None, 0, NULL_S) == -1
    assert ma(W, k, n, R(x), R(_t([k, m + 1])), R(nw), eps, R(_t([k, m])), R(y), None, 0, NULL_S) == -3
    assert ma(W, k, n, R(x), R(_t([k, m], BF16)), R(nw), eps, R(_t([k, m])), R(y), None, 0, NULL_S) == -2
    assert ma(W, k, n, R(x), R(_t([k, m])), R(nw), eps, R(x), R(y), None, 0, NULL_S) == -6   # sum aliases a
    # the AdaLN prologue: gate needs b, scale and shift come together, each F32 [k]
    md = L.mi_mul_mat_q8_0_adaln
    b2, s2 = _t([k, m]), _t([k, m])
    assert md(W, k, n, R(x), None, R(nw), R(nw), None, None, eps, None, R(y), None, 0, NULL_S) == -1  # gate, no b
    assert md(W, k, n, R(x), None, None, R(nw), R(nw), None, eps, None, R(y), None, 0, NULL_S) == -1  # scale alone
    assert md(W, k, n, R(x), None, None, R(nw), None, R(nw), eps, None, R(y), None, 0, NULL_S) == -1  # shift alone
    assert md(W, k, n, R(x), R(b2), R(nw), R(nw), None, None, eps, None, R(y), None, 0, NULL_S) == -1  # b, no sum
    assert md(W, k, n, R(x), R(b2), R(_t([k + 32])), R(nw), None, None, eps, R(s2), R(y), None, 0, NULL_S) == -3
    assert md(W, k, n, R(x), R(b2), R(_t([k], BF16)), R(nw), None, None, eps, R(s2), R(y), None, 0, NULL_S) == -2
    assert md(W, k, n, R(x), None, None, R(nw), R(_t([k, 2])), R(nw), eps, None, R(y), None, 0, NULL_S) == -3
    assert md(W, k, n, R(x), None, None, R(nw), R(nw), R(_t([k], BF16)), eps, None, R(y), None, 0, NULL_S) == -2
    assert md(W, k, n, R(x), R(b2), R(nw), R(nw), R(nw), R(nw), eps, R(b2), R(y), None, 0, NULL_S) == -6  # sum aliases b
    assert md(W, k, n, R(x), R(b2), R(nw), R(nw), R(nw), R(nw), eps, R(s2), R(y), None, 0, NULL_S) == -6  # no workspace
    # the SwiGLU prologue: gu [2k, m]
    gu = _t([2 * k, m])
    mg = L.mi_mul_mat_q8_0_swiglu
    assert L.mi_mul_mat_q8_0_swiglu_workspace(k, n, R(gu), ctypes.byref(nb)) == 0 and nb.value > 0
    wsn = nb.value
    assert L.mi_mul_mat_q8_0_workspace(k, n, R(x), ctypes.byref(nb)) == 0 and nb.value == wsn  # as for x [k, m]
    assert L.mi_mul_mat_q8_0_swiglu_workspace(k, n, R(gu), None) == -1
    assert L.mi_mul_mat_q8_0_swiglu_workspace(k, n, None, ctypes.byref(nb)) == -1
    assert mg(W, k, n, R(_t([2 * k + 2, m])), 0, R(y), None, 0, NULL_S) == -3     # not 2k wide
    assert mg(W, k, n, R(_t([2 * k, m], BF16)), 0, R(y), None, 0, NULL_S) == -2
    assert mg(W, k, n, R(gu), 0, R(_t([n, m + 1])), None, 0, NULL_S) == -3         # y rows
    assert mg(W, k, n, R(gu), 0, None, None, 0, NULL_S) == -1
    assert mg(W, k, n, R(gu), 1, R(y), ctypes.c_void_p(1 << 20), wsn - 1, NULL_S) == -6
    assert mg(W, k, n, R(gu), 1, R(y), ctypes.c_void_p((1 << 20) + 16), wsn, NULL_S) == -5
    # with the residual add after it: r F32 of y's shape; clamp bounds ordered
    mr = L.mi_mul_mat_q8_0_swiglu_add
    lo, hi = ctypes.c_float(-65504.0), ctypes.c_float(65504.0)
    r = _t([n, m])
    assert mr(W, k, n, R(gu), 0, None, 0, lo, hi, R(y), None, 0, NULL_S) == -1
    assert mr(W, k, n, R(gu), 0, R(r), 0, lo, hi, None, None, 0, NULL_S) == -1
    assert mr(W, k, n, R(gu), 0, R(_t([n, m], BF16)), 0, lo, hi, R(y), None, 0, NULL_S) == -2
    assert mr(W, k, n, R(gu), 0, R(_t([n, m + 1])), 0, lo, hi, R(y), None, 0, NULL_S) == -3
    assert mr(W, k, n, R(gu), 0, R(r), 1, hi, lo, R(y), None, 0, NULL_S) == -6     # lo > hi
    assert mr(W, k, n, R(gu), 0, R(r), 1, lo, hi, R(y), ctypes.c_void_p(1 << 20), wsn - 1, NULL_S) == -6
    assert mr(W, k, n, R(gu), 0, R(r), 1, lo, hi, R(y), ctypes.c_void_p((1 << 20) + 16), wsn, NULL_S) == -5
    # with the gated residual: gate F32 [n]
    mgg = L.mi_mul_mat_q8_0_swiglu_gated_add
    gv = _t([n])
    assert mgg(W, k, n, R(gu), 0, R(r), None, R(y), None, 0, NULL_S) == -1
    assert mgg(W, k, n, R(gu), 0, None, R(gv), R(y), None, 0, NULL_S) == -1
    assert mgg(W, k, n, R(gu), 0, R(r), R(_t([n + 1])), R(y), None, 0, NULL_S) == -3
    assert mgg(W, k, n, R(gu), 0, R(r), R(_t([n], BF16)), R(y), None, 0, NULL_S) == -2
    assert mgg(W, k, n, R(gu), 0, R(r), R(gv), R(y), ctypes.c_void_p(1 << 20), wsn - 1, NULL_S) == -6


def test_sampler_validation():
    oc, t, n = 64, 100, 2
    c = _t([oc, t, n])
    nb = ctypes.c_size_t(0)
    M = ctypes.c_void_p(1 << 20)
    assert L.mi_apg_buffer_bytes(R(c), ctypes.byref(nb)) == 0 and nb.value == oc * t * n * 8
    apg = L.mi_apg_forward
    assert apg(R(c), R(_t([oc, t + 1, n])), 3.0, -0.75, 2.5, M, nb.value, 1, R(c), NULL_S) == -3
    assert apg(R(c), R(c), 3.0, -0.75, 2.5, M, nb.value, 1, R(_t([oc, t, n], BF16)), NULL_S) == -2
    assert apg(R(c), R(c), float("inf"), -0.75, 2.5, M, nb.value, 1, R(c), NULL_S) == -6
    assert apg(R(c), R(c), 3.0, -0.75, 2.5, None, 0, 1, R(c), NULL_S) == -6           # no momentum buffer
    assert apg(R(c), R(c), 3.0, -0.75, 2.5, M, nb.value - 8, 1, R(c), NULL_S) == -6
    assert apg(R(c), R(c), 3.0, -0.75, 2.5, ctypes.c_void_p((1 << 20) + 4), nb.value, 1, R(c), NULL_S) == -5
    big = _t([1100, 2, 1])
    assert apg(R(big), R(big), 3.0, -0.75, 2.5, M, 1 << 30, 1, R(big), NULL_S) == -7  # more than 1024 channels
    strided = _t([oc, t, n], nb=[4, oc * 8, oc * 8 * t, oc * 8 * t * n])
    assert apg(R(strided), R(strided), 3.0, -0.75, 2.5, M, nb.value, 1, R(strided), NULL_S) == -4
    st = L.mi_flow_step
    assert st(7, R(c), R(c), 1.0, 0.5, 0, None, None, NULL_S) == -6                  # unknown solver
    assert st(0, R(c), R(c), 1.0, float("nan"), 0, None, None, NULL_S) == -6
    assert st(1, R(c), R(c), 1.0, 0.5, 3, R(c), R(c), NULL_S) == -6                  # history 0..2
    assert st(1, R(c), R(c), 1.0, 0.5, 0, None, R(c), NULL_S) == -1                  # dpm3m needs prev
    assert st(0, R(c), R(_t([oc, t, n + 1])), 1.0, 0.5, 0, None, None, NULL_S) == -3
    assert L.mi_flow_final(R(c), R(c), float("inf"), R(c), NULL_S) == -6


def _rock4(ms, fpa_rows=None, recf_len=None):
    ms = (ctypes.c_int32 * len(ms))(*ms)
    nrec = recf_len if recf_len is not None else sum(2 * m - 1 for m in ms)
    fpa = (ctypes.c_double * (6 * len(ms)))()
    fpb = (ctypes.c_double * (4 * len(ms)))()
    recf = (ctypes.c_double * max(nrec, 1))()
    tab = _lib.MiRock4Tables(ctypes.cast(ms, ctypes.POINTER(ctypes.c_int32)),
                             ctypes.cast(fpa, ctypes.POINTER(ctypes.c_double)),
                             ctypes.cast(fpb, ctypes.POINTER(ctypes.c_double)),
                             ctypes.cast(recf, ctypes.POINTER(ctypes.c_double)), len(ms), nrec)
    tab._keep = (ms, fpa, fpb, recf)
    return tab


def test_other_solvers_validation():
    oc, t, n = 64, 100, 2
    c = _t([oc, t, n])
    sde = L.mi_flow_step_sde
    assert sde(R(c), R(c), R(_t([oc, t, n + 1])), 1.0, 0.5, NULL_S) == -3          # noise shape
    assert sde(R(c), R(c), R(_t([oc, t, n], BF16)), 1.0, 0.5, NULL_S) == -2
    assert sde(R(c), R(c), R(c), float("nan"), 0.5, NULL_S) == -6
    nb = ctypes.c_size_t(0)
    assert L.mi_stork4_workspace(R(c), ctypes.byref(nb)) == 0 and nb.value >= oc * t * n * 4
    W = ctypes.c_void_p(1 << 20)
    st = L.mi_stork4_step
    tab = _rock4([1, 2, 4, 10, 20])
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 10, None, W, nb.value, NULL_S) == -1
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 10, R(tab), None, 0, NULL_S) == -6
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 10, R(tab), W, nb.value - 4, NULL_S) == -6
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 10, R(tab), ctypes.c_void_p((1 << 20) + 64),
              nb.value, NULL_S) == -5
    assert st(R(c), R(c), 1.0, 0.9, -1, 0.1, 0.0, R(c), R(c), 10, R(tab), W, nb.value, NULL_S) == -6
    assert st(R(c), R(c), 1.0, float("inf"), 1, 0.1, 0.0, R(c), R(c), 10, R(tab), W, nb.value, NULL_S) == -6
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(_t([oc, t + 1, n])), R(c), 10, R(tab), W, nb.value,
              NULL_S) == -3
    bad = _rock4([1, 4, 2])                                                        # degrees not ascending
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 10, R(bad), W, nb.value, NULL_S) == -6
    big = _rock4([2, 200])                                                         # degree above 160
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 10, R(big), W, nb.value, NULL_S) == -7
    short = _rock4([1, 2, 4, 10, 20], recf_len=30)                                 # recf too short for 20
    assert st(R(c), R(c), 1.0, 0.9, 1, 0.1, 0.0, R(c), R(c), 20, R(short), W, nb.value, NULL_S) == -6
    dcw = L.mi_dcw
    assert dcw(4, R(c), R(c), 0.5, 0.4, 0.3, 0.0, NULL_S) == -6                     # unknown mode
    assert dcw(0, R(c), R(_t([oc, t, n + 1])), 0.5, 0.4, 0.3, 0.0, NULL_S) == -3
    assert dcw(0, R(c), R(c), 0.5, 0.4, float("nan"), 0.0, NULL_S) == -6
    assert dcw(0, R(c), R(c), 0.5, 0.4, 0.0, 0.7, NULL_S) == 0                      # low band scaler 0: no launch


def test_chain_validation():
    io = _lib.MiDitBlockIO()
    io.hidden = _t([2048, 4])
    io.adaln = _t([2048 * 5])
    assert L.mi_dit_block_ops(R(io), NULL_S) == -3
    assert L.mi_dit_block_ops(None, NULL_S) == -1
    assert L.mi_qwen3_layer_ops(None, NULL_S) == -1


def test_descriptor_extent_overflow_is_refused():
    """ne1*ne2*ne3 (or the byte extent) past int64 is refused before launch:
    an unchecked product would wrap to a small or negative row count."""
    y = _t([4, 8])
    wrap = _t([4, 2**32 + 1, 2**32 - 1, 1], nb=[4, 16, 16, 16])   # rows wrap to -1 in int64
    assert L.mi_rms_norm(R(wrap), None, 1e-6, R(y), NULL_S) in (-3, -7)
    big = _t([4, 2**20, 2**20, 2**20], nb=[4, 16, 16, 16])          # 2^60 rows x 4: elements overflow
    assert L.mi_rms_norm(R(big), None, 1e-6, R(y), NULL_S) in (-3, -7)
    ext = _t([4, 2, 1, 1], nb=[4, 2**63 - 8, 16, 16])               # byte extent past 2^63
    assert L.mi_rms_norm(R(ext), None, 1e-6, R(_t([4, 2])), NULL_S) == -7
    assert L.mi_rms_norm(R(_t([4, 2**31, 1, 1])), None, 1e-6, R(y), NULL_S) == -7


def _qwen3_io(**bad):
    """A decode-layer io (H=256, 4/2 heads x 64, I=512, 2 tokens, F32, Q8_0
    caches) over fake, never dereferenced addresses; `bad` replaces fields."""
    H, NH, NKV, D, I, N, SLOTS = 256, 4, 2, 64, 512, 2, 16
    addr = [1 << 40]

    def t(shape, typ=F32, nb=None):
        addr[0] += 1 << 30
        return _t(shape, typ, data=addr[0], nb=nb)

    qkv_row = (NH + 2 * NKV) * D * 4
    qkv = t([(NH + 2 * NKV) * D, N])
    view = lambda off, heads: _t([D, heads, N], data=qkv.data + off, nb=[4, D * 4, qkv_row, qkv_row * N])  # noqa
    io = _lib.MiQwen3LayerIO()
    io.hidden, io.in_norm_w, io.post_norm_w = t([H, N]), t([H]), t([H])
    io.norm, io.norm2 = t([H, N]), t([H, N])
    io.q, io.k, io.v = view(0, NH), view(NH * D * 4, NKV), view((NH + NKV) * D * 4, NKV)
    io.q_w, io.k_w, io.q_out, io.k_out, io.pos = t([D]), t([D]), t([D, NH, N]), t([D, NKV, N]), t([N], I32)
    io.k_cache, io.v_cache = t([D, SLOTS, NKV, N], Q8_0), t([D, SLOTS, NKV, N], Q8_0)
    io.pos0, io.sets = t([N], I32), t([N], I32)
    io.attn_out, io.gate_up, io.ff, io.mlp_out = t([H, N]), t([2 * I, N]), t([I, N]), t([H, N])
    io.eps, io.rope_freq_base, io.n_dims, io.clamp_fp16, io.kv_rounding = 1e-6, 1e6, D, 1, _lib.Q8_0_CPU_X86
    for k, v in bad.items():
        setattr(io, k, v)
    return io


def test_chain_drivers_validate_before_any_launch():
    """A bad operand late in the chain is reported as such (-3), not as the
    HIP error (-8) the first launch gives on this GPU-less host: the whole
    chain is validated before anything is launched (and so before `hidden`
    could be updated in place)."""
    assert L.mi_qwen3_layer_ops(R(_qwen3_io(mlp_out=_t([255, 2], data=1 << 50))), NULL_S) == -3
    assert L.mi_qwen3_layer_ops(R(_qwen3_io(ff=_t([511, 2], data=1 << 50))), NULL_S) == -3
    assert L.mi_qwen3_layer_ops(R(_qwen3_io(attn_out=_t([256, 3], data=1 << 50))), NULL_S) == -3
    no_kout = _qwen3_io(k_out=_t([64, 2, 2], data=0), n_dims=32)     # fused path: partial rotation refused
    assert L.mi_qwen3_layer_ops(R(no_kout), NULL_S) == -7


def test_product_path_has_no_fallback(tmp_path):
    """The ops fail loudly when the HIP library is absent (no CPU fallback)."""
    import subprocess
    import sys

    code = ("import sys; sys.path.insert(0, %r)\n"
            "import acestep_ops\n"
            "try:\n    acestep_ops.load()\nexcept ImportError as e:\n    print('IMPORT-ERROR', e); sys.exit(3)\n"
            "sys.exit(0)\n") % os.path.join(ROOT, "hbd-acestep.cpp_amd")
    env = dict(os.environ, MI_OPS_LIB=str(tmp_path / "missing.so"))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 3 and "IMPORT-ERROR" in r.stdout
