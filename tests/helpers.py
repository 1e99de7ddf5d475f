"""Shared test helpers: tolerance checks, bf16 plumbing, seeded inputs."""
from __future__ import annotations

import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def rng(seed: int = 42):
    return np.random.default_rng(seed)


def randn(shape, seed=42, scale=1.0, mean=0.0):
    return (rng(seed).standard_normal(shape) * scale + mean).astype(np.float32)


# ---------------------------------------------------------------------------
# tolerances (the bars stated for this path)
#   fp32: max relative error <= 1e-5; where an output is a difference that can
#         cancel (rope, modulate, gated add) the denominator is floored at the
#         RMS of the reference row: |a-b| <= 1e-5 * max(|ref|, rms(ref row)).
#   bf16: within 1 bf16 ulp of the oracle's RNE-rounded fp32 result; for
#         outputs that are differences that can cancel (rope, modulate), an
#         element beyond 1 ulp must still meet the fp32 bar with the row floor,
#         |a-b| <= 1e-5 * rms(ref row): near zero a bf16 ulp is far below the
#         fp32 rounding of the terms that cancelled.
# ---------------------------------------------------------------------------
def rel_err(a: np.ndarray, ref: np.ndarray, row_floor: bool = False, tiny: float = 1e-30) -> float:
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref)
    if row_floor:
        rms = np.sqrt(np.mean(ref.reshape(-1, ref.shape[-1]) ** 2, axis=-1, keepdims=True))
        den = np.maximum(den.reshape(-1, ref.shape[-1]), rms).reshape(ref.shape)
    den = np.maximum(den, tiny)
    both_nan = np.isnan(a) & np.isnan(ref)
    same_inf = np.isinf(a) & np.isinf(ref) & (np.sign(a) == np.sign(ref))
    with np.errstate(invalid="ignore"):
        e = np.abs(a - ref) / den
    e[both_nan | same_inf] = 0.0
    return float(np.max(e)) if e.size else 0.0


def assert_f32_close(a, ref, tol=1e-5, row_floor=False):
    e = rel_err(a, ref, row_floor=row_floor)
    assert e <= tol, f"max relative error {e:.3e} > {tol:.1e}"
    return e


def bf16_ordinal(h: np.ndarray) -> np.ndarray:
    """Monotone integer index of bf16 bit patterns (adjacent values differ by 1)."""
    h = np.asarray(h, np.uint16).astype(np.int64)
    mag = h & 0x7FFF
    return np.where(h & 0x8000, -mag, mag)


def assert_bf16_ulp(a_bits, ref_bits, max_ulp=1, row_floor=False, tol=1e-5):
    d = np.abs(bf16_ordinal(a_bits) - bf16_ordinal(ref_bits))
    bad = d > max_ulp
    if row_floor and bad.any():
        a = (np.asarray(a_bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        r = (np.asarray(ref_bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        n = r.shape[-1]
        rms = np.sqrt(np.mean(r.reshape(-1, n) ** 2, axis=1, keepdims=True))
        floor = (tol * rms * np.ones((1, n))).reshape(r.shape)
        bad &= ~(np.abs(a - r) <= floor)
    worst = int(d[bad].max()) if bad.any() else 0
    assert not bad.any(), f"{int(bad.sum())} elements beyond {max_ulp} bf16 ulp (worst {worst})"
    return int(d.max()) if d.size else 0


def assert_mul_mat_q8_0(y, w, x):
    """ggml_mul_mat with Q8_0 weights w (n, k/32*34 bytes) and F32 x (m, k): the
    exact value of ggml-cpu's definition (x quantized with the x86 Q8_0
    quantizer, exact int32 block dots scaled by fp16(d_w) fp16(d_x)), and the
    kernels' rounding bound: one rounding per block (fma into the running sum)
    and per added split, |y - ref| <= (K/32 + 8) 2^-24 sum_k |w_k| |x'_k|."""
    from oracle import oracle as orc

    ref = orc.mul_mat_q8_0(w, x)
    k = x.shape[-1]
    wf = orc.dequantize_q8_0(w).astype(np.float64)
    xf = orc.dequantize_q8_0(orc.quantize_q8_0(x, "x86")).astype(np.float64)
    bound = (k / 32 + 8) * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T) + 1e-30
    err = np.abs(np.asarray(y, np.float64) - ref)
    assert y.shape == ref.shape
    assert np.all(err <= bound), f"max err {err.max()} vs bound {bound[err > bound].min()}"


def frac_bitexact(a: np.ndarray, ref: np.ndarray) -> float:
    a = np.ascontiguousarray(a)
    ref = np.ascontiguousarray(ref)
    eq = a.view(np.uint8).reshape(a.size, -1) == ref.view(np.uint8).reshape(ref.size, -1)
    return float(np.mean(np.all(eq, axis=1)))


def tsembd_bar(y, ref, t, dim, max_period):
    """1e-5 relative (row-RMS floor) plus the conditioning of cos/sin(t*freq):
    a 1-ulp difference between device and glibc exp in freq moves the angle by
    |t*freq| * 2^-23, which no implementation can avoid at t ~ 1000."""
    half = dim // 2
    freq = np.exp(-np.log(max_period) * np.arange(half) / half)
    arg = np.abs(t.astype(np.float64)[:, None] * freq[None, :])
    slack = np.concatenate([arg, arg], axis=1) * 2.0 ** -23
    if dim % 2:
        slack = np.concatenate([slack, np.zeros((t.size, 1))], axis=1)
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=1, keepdims=True))
    bound = 1e-5 * np.maximum(np.abs(ref), rms) + slack
    worst = np.max(np.abs(y.astype(np.float64) - ref) - bound)
    assert worst <= 0, f"timestep embedding exceeds bound by {worst:.3e}"


# ---------------------------------------------------------------------------
# host <-> device (acestep_ops.device; bf16/f16 travel as uint16 bit patterns)
# ---------------------------------------------------------------------------
def to_dev(a: np.ndarray, dev=None, bf16: bool = False, f16: bool = False):
    from acestep_ops.device import DTensor

    if bf16 or f16:
        assert a.dtype in (np.uint16, np.int16)
        return DTensor.from_numpy(a.view(np.uint16), "bf16" if bf16 else "f16")
    return DTensor.from_numpy(np.ascontiguousarray(a))


def to_np(t) -> np.ndarray:
    return t.numpy()
