"""acestep_ops -- MI355X (gfx950) per-layer fused ops of acestep.cpp's Qwen3 LM
and ACE-Step DiT graph builders, behind the C ABI of include/mi_ops.h.

``acestep_ops.ops`` holds one wrapper per entry point (ggml op names) over
``device.DTensor`` views;
``acestep_ops._lib`` the ctypes binding. The HIP library is the only compute
path; importing the ops without the built library raises ImportError.
"""
from ._lib import BF16, F16, F32, I32, LIB_PATH, Q8_0, Q8_0_CPU_X86, Q8_0_REF, MiError, load  # noqa: F401

__all__ = ["load", "MiError", "LIB_PATH", "F32", "F16", "BF16", "Q8_0", "I32", "Q8_0_CPU_X86", "Q8_0_REF"]
