"""ctypes binding of libmi_ops.so (the C ABI in include/mi_ops.h).

The shared library is built in-tree (``make -C hbd-acestep.cpp_amd``) and is
the only compute path: if it cannot be loaded, importing this module raises.
"""
from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.normpath(os.path.join(_PKG_DIR, "..", "lib"))
LIB_PATH = os.environ.get("MI_OPS_LIB", os.path.join(LIB_DIR, "libmi_ops.so"))

# enum mi_type (values equal enum ggml_type)
F32, F16, Q8_0, I32, BF16 = 0, 1, 8, 26, 30
# enum mi_q8_0_rounding
Q8_0_CPU_X86, Q8_0_REF = 0, 1

NOALLOC_SCRATCH_BYTES = 32 << 20  # MI_MUL_MAT_NOALLOC_SCRATCH_BYTES

STATUS = {
    0: "MI_OK",
    -1: "MI_ERR_NULL",
    -2: "MI_ERR_TYPE",
    -3: "MI_ERR_SHAPE",
    -4: "MI_ERR_STRIDE",
    -5: "MI_ERR_ALIGN",
    -6: "MI_ERR_PARAM",
    -7: "MI_ERR_UNSUPPORTED",
    -8: "MI_ERR_HIP",
    -9: "MI_ERR_FILE",
    -10: "MI_ERR_SCRATCH",
}


class MiTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_uint64 * 4),
    ]


_TP = ctypes.POINTER(MiTensor)
_VP = ctypes.c_void_p
_F = ctypes.c_float
_I = ctypes.c_int


class MiGGUFTensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("type", ctypes.c_int32),
        ("n_dims", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nbytes", ctypes.c_uint64),
        ("data", ctypes.c_void_p),
    ]


class MiDitBlockIO(ctypes.Structure):
    _fields_ = [(n, MiTensor) for n in (
        "hidden", "adaln", "sa_norm_w", "ffn_norm_w", "norm_sa",
        "q", "k", "q_w", "k_w", "q_out", "k_out", "pos",
        "sa_out", "ca_norm_w", "norm_ca", "ca_q", "ca_q_w", "ca_q_out", "ca_out", "ca_k", "ca_k_w", "ca_k_out",
        "norm_ffn", "gate_up", "ff", "ffn_out")] + [
        ("eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float),
        ("n_dims", ctypes.c_int), ("use_cross_attn", ctypes.c_int)]


class MiRock4Tables(ctypes.Structure):
    _fields_ = [("ms", ctypes.POINTER(ctypes.c_int32)), ("fpa", ctypes.POINTER(ctypes.c_double)),
                ("fpb", ctypes.POINTER(ctypes.c_double)), ("recf", ctypes.POINTER(ctypes.c_double)),
                ("ms_len", ctypes.c_int32), ("recf_len", ctypes.c_int32)]


class MiQwen3LayerIO(ctypes.Structure):
    _fields_ = [(n, MiTensor) for n in (
        "hidden", "in_norm_w", "post_norm_w", "norm", "norm2",
        "q", "k", "v", "q_w", "k_w", "q_out", "k_out", "pos",
        "k_cache", "v_cache", "pos0", "sets", "attn_out", "gate_up", "ff", "mlp_out")] + [
        ("eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float), ("n_dims", ctypes.c_int),
        ("clamp_fp16", ctypes.c_int), ("kv_rounding", ctypes.c_int), ("d_err", ctypes.c_void_p)]


# name -> argtypes, exactly the prototypes of include/mi_ops.h
PROTOTYPES = {
    "mi_abi_version": [],
    "mi_status_str": [_I],
    "mi_rms_norm": [_TP, _TP, _F, _TP, _VP],
    "mi_rms_norm_modulate": [_TP, _TP, _TP, _TP, _F, _TP, _VP],
    "mi_add_rms_norm": [_TP, _TP, _TP, _I, _F, _F, _TP, _TP, _TP, _F, _TP, _TP, _VP],
    "mi_rope_ext": [_TP, _TP, _I, _I, _F, _F, _F, _F, _TP, _VP],
    "mi_qk_norm_rope": [_TP, _TP, _TP, _TP, _TP, _TP, _TP, _F, _I, _F, _F, _F, _VP],
    "mi_swiglu": [_TP, _I, _TP, _VP],
    "mi_swiglu_split": [_TP, _TP, _TP, _VP],
    "mi_add": [_TP, _TP, _TP, _VP],
    "mi_mul": [_TP, _TP, _TP, _VP],
    "mi_add_clamp": [_TP, _TP, _F, _F, _TP, _VP],
    "mi_gated_add": [_TP, _TP, _TP, _TP, _VP],
    "mi_modulate": [_TP, _TP, _TP, _TP, _VP],
    "mi_get_rows": [_TP, _TP, _TP, _VP, _VP],
    "mi_cpy": [_TP, _TP, _VP],
    "mi_cpy_q8_0": [_TP, _TP, _I, _VP],
    "mi_kv_store": [_TP, _TP, _TP, _TP, _TP, _TP, _I, _VP, _VP],
    "mi_qk_norm_rope_kv_store": [_TP, _TP, _TP, _TP, _TP, _TP, _TP, _F, _I, _F, _F, _F, _I, _TP, _TP, _TP, _TP, _I,
                                 _VP, _VP],
    "mi_scale": [_TP, _F, _TP, _VP],
    "mi_timestep_embedding": [_TP, _I, _I, _TP, _VP],
    "mi_flash_attn_ext_workspace": [_TP, _TP, _TP, ctypes.POINTER(ctypes.c_size_t)],
    "mi_flash_attn_ext": [_TP, _TP, _TP, _TP, _F, _F, _F, _TP, _VP, ctypes.c_size_t, _VP],
    "mi_q8_0_repack_bytes": [ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ctypes.c_size_t)],
    "mi_q8_0_repack": [_TP, _VP, ctypes.c_size_t, _VP],
    "mi_mul_mat_q8_0_workspace": [ctypes.c_int64, ctypes.c_int64, _TP, ctypes.POINTER(ctypes.c_size_t)],
    "mi_mul_mat_q8_0": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, _TP, _VP, ctypes.c_size_t, _VP],
    "mi_mul_mat_q8_0_noalloc": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, _TP, _VP],
    "mi_mul_mat_q8_0_rms_norm": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, _TP, ctypes.c_float, _TP, _VP,
                                 ctypes.c_size_t, _VP],
    "mi_mul_mat_q8_0_add_rms_norm": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, _TP, _TP, ctypes.c_float, _TP, _TP,
                                     _VP, ctypes.c_size_t, _VP],
    "mi_mul_mat_q8_0_adaln": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, _TP, _TP, _TP, _TP, _TP, ctypes.c_float, _TP,
                              _TP, _VP, ctypes.c_size_t, _VP],
    "mi_mul_mat_q8_0_swiglu_workspace": [ctypes.c_int64, ctypes.c_int64, _TP, ctypes.POINTER(ctypes.c_size_t)],
    "mi_mul_mat_q8_0_swiglu": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, ctypes.c_int, _TP, _VP, ctypes.c_size_t,
                               _VP],
    "mi_mul_mat_q8_0_swiglu_add": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, ctypes.c_int, _TP, ctypes.c_int, _F, _F,
                                   _TP, _VP, ctypes.c_size_t, _VP],
    "mi_mul_mat_q8_0_swiglu_gated_add": [_VP, ctypes.c_int64, ctypes.c_int64, _TP, ctypes.c_int, _TP, _TP, _TP, _VP,
                                         ctypes.c_size_t, _VP],
    "mi_apg_buffer_bytes": [_TP, ctypes.POINTER(ctypes.c_size_t)],
    "mi_apg_forward": [_TP, _TP, _F, _F, _F, _VP, ctypes.c_size_t, _I, _TP, _VP],
    "mi_flow_step": [_I, _TP, _TP, _F, _F, _I, _TP, _TP, _VP],
    "mi_flow_final": [_TP, _TP, _F, _TP, _VP],
    "mi_flow_step_sde": [_TP, _TP, _TP, _F, _F, _VP],
    "mi_stork4_workspace": [_TP, ctypes.POINTER(ctypes.c_size_t)],
    "mi_stork4_step": [_TP, _TP, _F, _F, _I, _F, _F, _TP, _TP, _I, ctypes.POINTER(MiRock4Tables), _VP,
                       ctypes.c_size_t, _VP],
    "mi_dcw": [_I, _TP, _TP, _F, _F, _F, _F, _VP],
    "mi_gguf_open": [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)],
    "mi_gguf_close": [_VP],
    "mi_gguf_n_tensors": [_VP],
    "mi_gguf_find_tensor": [_VP, ctypes.c_char_p],
    "mi_gguf_get_tensor": [_VP, ctypes.c_int64, ctypes.POINTER(MiGGUFTensor)],
    "mi_gguf_n_kv": [_VP],
    "mi_gguf_find_key": [_VP, ctypes.c_char_p],
    "mi_gguf_get_key": [_VP, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int32)],
    "mi_gguf_get_u32": [_VP, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)],
    "mi_gguf_get_f32": [_VP, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)],
    "mi_gguf_get_bool": [_VP, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)],
    "mi_gguf_get_str": [_VP, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)],
    "mi_gguf_upload": [_VP, ctypes.c_char_p, _I, _VP, ctypes.c_size_t, _VP],
    "mi_gguf_upload_rows": [_VP, ctypes.POINTER(ctypes.c_char_p), _I, _VP, ctypes.c_size_t,
                            ctypes.POINTER(ctypes.c_int64), _VP],
    "mi_dit_block_ops": [ctypes.POINTER(MiDitBlockIO), _VP],
    "mi_qwen3_layer_ops": [ctypes.POINTER(MiQwen3LayerIO), _VP],
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libmi_ops.so; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libmi_ops.so not found at {LIB_PATH}; build it with `make -C hbd-acestep.cpp_amd` "
                          "(or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.mi_status_str.restype = ctypes.c_char_p
    for name in ("mi_gguf_n_tensors", "mi_gguf_find_tensor", "mi_gguf_n_kv", "mi_gguf_find_key"):
        getattr(lib, name).restype = ctypes.c_int64
    lib.mi_gguf_close.restype = None
    _lib = lib
    return lib


class MiError(RuntimeError):
    def __init__(self, fn: str, rc: int):
        msg = load().mi_status_str(rc).decode()
        super().__init__(f"{fn} failed: {STATUS.get(rc, rc)} ({msg})")
        self.rc = rc


def call(name: str, *args) -> None:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise MiError(name, rc)
