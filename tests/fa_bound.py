"""Error bound of the flash-attention kernels against the exact value, derived
from their arithmetic (fattn.hip), element by element.

The kernels compute y = sum_j p_j v_j / sum_j p_j with p_j = exp(x_j - m),
x_j = scale * (q'.k_j) + mask_j, in fp32 (q' = q converted to K's dot type, as
ggml-cpu converts it; the oracle converts it the same way). Writing each
computed p_j as p_j (1 + eta_j), the first-order change of y is
sum_j p_j eta_j (v_j - y) / l, so

  |y - ref| <= [sum_j p_j (eta_j + eta_r) (|v_j| + |ref|)] / l      (weights)
             + [sum_j |e_j| |v_j|] / l                                (16-bit P parts)
             + lambda sqrt(n) u [sum_j p_j |v_j| / l + |ref|]         (sums of o and l)
             + 2 u |ref|                                              (1 / l and the product)

with u = 2^-24 and, per key,
  eta_j = c u |scale| sum_d |q'_d k_jd|     the dot product: at most c roundings of
                                            partial sums bounded by sum |q' k|; c = D
                                            (fdot2 / fma chains, 32x32x16 MFMA chains),
                                            D/32 + 3 for Q8_0 K (exact int32 blocks, one
                                            product and one fma per block)
        + 3 u (|x_j| + |x_j - m| + |m|)     scale, mask add, max shift, the log2 e factor
        + 4 u                               exp / exp2 (v_exp_f32, 1 ulp)
and per row eta_r = 3 u (max x - min x) + 2 u (n_kv / 32 + 2): the running-max
rescales (each exp(m_old - m_new) carries the error above; their arguments add
up to at most the score range) and the split merge weights.
e_j: the matrix-core path multiplies V by P split into a high and a low 16-bit
part while l sums the fp32 p. With u_h the unit roundoff of the 16-bit type
(2^-8 bf16, 2^-11 fp16), |p - hi| <= u_h p, and the low part rounds that
remainder, which lies at least one binade lower: |e_j| <= 2^-17 p_j for bf16
parts (reached: p = 1 + 2^-9 + 2^-17 keeps 1 + 2^-9), 2^-22 p_j + 2^-25 for
fp16 parts (the low part may be subnormal). Over a Q8_0 cache the decode
kernel splits p_j d_v (rounded once) into bf16 parts and multiplies the
quants: relative to p_j |v_j| that is 2^-17 + 2^-24. The Q8_0 prefill kernel
holds V' = q d_v exactly as a bf16 high part V_h and an fp16 low part V_l
(|V_l| <= 2^-8 |V'|) and forms (P_hi + P_lo) V_h + RN_fp16(p) V_l: relative to
p_j |v_j|, 2^-17 (1 + 2^-8) + 2^-11 2^-8, plus 2^-25 2^-8 |v_j| for a
subnormal fp16 p.
The accumulation of o and l over n = n_kv (+ 2 n_kv for the two MFMA passes,
3 n_kv for the Q8_0 prefill kernel's three)
roundings uses the probabilistic bound of Higham and Mary (SIAM J. Sci.
Comput. 41(5), 2019): with rounding errors independent and mean zero, the
error of an n-term sum is at most lambda sqrt(n) u sum |terms| with
probability >= 1 - 2 exp(-lambda^2 (1 - u)^2 / 2) per element; lambda = 8
(failure probability below 1e-13). Everything else is worst case.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc

U = 2.0 ** -24
LAMBDA = 8.0


def convert_q(q, kt: str):
    """q as ggml-cpu converts it to K's vec_dot type (float values)."""
    if kt == "f16":
        return orc.f16_to_f32(orc.f32_to_f16(q))
    if kt == "bf16":
        return orc.bf16_to_f32(orc.f32_to_bf16(q))
    if kt == "q8_0":
        D = q.shape[-1]
        return orc.dequantize_q8_0(orc.quantize_q8_0(np.ascontiguousarray(q).reshape(-1, D), "x86")).reshape(q.shape)
    return q


def fa_bound(q, k, v, mask, scale: float, kt: str, mfma=False):
    """q (N, Nh, n_q, D) as handed to the kernel; k, v (Nk3, Nkv, n_kv, D) float
    values of the stored K/V; mask (mN, mH, mQ, n_kv) float values or None.
    mfma: False for the split path, True or "dec" for a matrix-core kernel
    (over a Q8_0 cache: the decode kernel), "prefill" for the matrix-core
    prefill kernel (the two differ only over a Q8_0 cache).
    Returns the bound (N, n_q, Nh, D) (NaN where every key is masked)."""
    N, Nh, n_q, D = q.shape
    Nk3, Nkv, n_kv, _ = k.shape
    rk, rk3 = Nh // Nkv, N // Nk3
    qc = convert_q(np.asarray(q, np.float32), kt).astype(np.float64)
    c = D / 32 + 3 if kt == "q8_0" else D
    q8_prefill = kt == "q8_0" and mfma == "prefill"
    n_round = ((4 if q8_prefill else 3) * n_kv if mfma else n_kv) + 64
    out = np.empty((N, n_q, Nh, D))
    for b in range(N):
        for g in range(Nkv):
            K = k[b // rk3, g].astype(np.float64)
            V = v[b // rk3, g].astype(np.float64)
            aV = np.abs(V)
            hs = range(g * rk, (g + 1) * rk)
            Q = np.stack([qc[b, h] for h in hs])                       # (rk, n_q, D)
            dots = Q @ K.T                                              # (rk, n_q, n_kv)
            A = np.abs(Q) @ np.abs(K).T
            if mask is not None:
                mN, mH = mask.shape[0], mask.shape[1]
                M = np.stack([mask[b % mN, h % mH, :n_q].astype(np.float64) for h in hs])
            else:
                M = np.zeros_like(dots)
            live = M != -np.inf
            x = np.where(live, scale * dots + np.where(live, M, 0.0), -np.inf)
            m = x.max(axis=-1, keepdims=True)
            ok = np.isfinite(m)
            ms = np.where(ok, m, 0.0)
            p = np.where(live, np.exp(np.where(live, x, ms) - ms), 0.0)
            lsum = p.sum(axis=-1, keepdims=True)
            ref = (p @ V) / np.where(lsum > 0, lsum, 1.0)
            xl = np.where(live, x, 0.0)
            eta = c * U * abs(scale) * A + 3 * U * (np.abs(xl) + np.abs(xl - ms) + np.abs(ms)) + 4 * U
            xmin = np.where(live, x, np.inf).min(axis=-1, keepdims=True)
            eta_r = 3 * U * np.where(ok, m - xmin, 0.0) + 2 * U * (n_kv / 32 + 2)
            w = p * (eta + eta_r)
            L = np.where(lsum > 0, lsum, 1.0)
            t1 = (w @ aV + np.abs(ref) * w.sum(axis=-1, keepdims=True)) / L
            t3 = LAMBDA * np.sqrt(n_round) * U * ((p @ aV) / L + np.abs(ref))
            bound = t1 + t3 + 2 * U * np.abs(ref) + 1e-37
            if mfma:
                if kt == "bf16":
                    e = p * 2.0 ** -17
                elif q8_prefill:
                    e = p * (2.0 ** -17 + 2.0 ** -19 + 2.0 ** -24) + np.where(live, 2.0 ** -33, 0.0)
                elif kt == "q8_0":
                    e = p * (2.0 ** -17 + U)
                else:
                    e = p * 2.0 ** -22 + np.where(live, 2.0 ** -25, 0.0)
                bound = bound + (e @ aV) / L
            bound = np.where(ok, bound, np.nan)
            for i, h in enumerate(hs):
                out[b, :, h] = bound[i]
    return out
