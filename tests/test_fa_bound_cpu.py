"""The flash-attention error bound (tests/fa_bound.py) against fp32 emulations
of the kernels' arithmetic on the CPU: the split-key path (sequential fp32 dot
products, tile-wise running max with rescales, fp32 accumulation of o and l),
the matrix-core path (P as high + low 16-bit parts in the p.V product, l
from the fp32 p), and the Q8_0 decode and prefill kernels. Each emulation must stay inside the bound, including at
large score magnitudes where exp amplifies score errors; and the bound must
not be vacuous (a wrong weight or a dropped rescale exceeds it)."""
import numpy as np
import pytest
from fa_bound import convert_q, fa_bound
from oracle import oracle as orc

F = np.float32


def _emulate(q, k, v, mask, scale, kt, mfma=False, tile=32, drop_rescale=False):
    """One (b, head) pair per row; k, v (1, 1, n_kv, D)."""
    qc = convert_q(q, kt).astype(F)[0]          # (Nh, n_q, D)
    K, V = k[0, 0].astype(F), v[0, 0].astype(F)
    Nh, n_q, D = qc.shape
    n_kv = K.shape[0]
    y = np.empty((1, n_q, Nh, D), F)
    for h in range(Nh):
        for iq in range(n_q):
            m, l, o = F(-np.inf), F(0), np.zeros(D, F)
            for t0 in range(0, n_kv, tile):
                kk = slice(t0, min(n_kv, t0 + tile))
                s = np.zeros(kk.stop - kk.start, F)
                for d in range(D):                     # sequential fp32 dot (fma-like: products exact)
                    s = F(s + qc[h, iq, d] * K[kk, d])
                mv = mask[0, 0, iq, kk] if mask is not None else np.zeros_like(s)
                x = np.where(mv == -np.inf, F(-np.inf), F(F(s * F(scale)) + mv)).astype(F)
                mn = F(max(m, x.max()))
                if mn == -np.inf:
                    continue
                alpha = F(1) if drop_rescale else F(np.exp(F(m - mn)))
                p = np.exp((x - mn).astype(F)).astype(F)
                if mfma:
                    cv = orc.f32_to_bf16 if kt == "bf16" else orc.f32_to_f16
                    bk = orc.bf16_to_f32 if kt == "bf16" else orc.f16_to_f32
                    hi = bk(cv(p))
                    lo = bk(cv((p - hi).astype(F)))
                    pv = (hi.astype(np.float64) + lo).astype(F)
                else:
                    pv = p
                m = mn
                l = F(l * alpha)
                o = (o * alpha).astype(F)
                for j in range(p.size):                # sequential fp32 accumulation
                    l = F(l + p[j])
                    o = (o + pv[j] * V[kk.start + j]).astype(F)
            y[0, iq, h] = (o * F(F(1) / l)).astype(F)
    return y


def _q8_parts(x):
    """Q8_0 (x86) of rows x (..., D): block scales (..., D/32) and quants (..., D), as floats."""
    D = x.shape[-1]
    b = orc.quantize_q8_0(np.ascontiguousarray(x, F).reshape(-1, D), "x86").reshape(-1, D // 32, 34)
    d = b[:, :, :2].copy().view(np.float16)[..., 0].astype(F)
    qs = b[:, :, 2:].view(np.int8).astype(F)
    return d.reshape(x.shape[:-1] + (D // 32,)), qs.reshape(x.shape)


def _emulate_q8_dec(q, k, v, mask, scale, tile=32):
    """The Q8_0 matrix-core decode kernel's arithmetic: q and K, V as Q8_0 (k, v
    hold the float rows the quantizer sees), exact int block dots scaled by
    fma(d_k * d_q, dot, s) with blocks 0-1 and 2-3 summed apart, p.V as
    (p * d_v) split into bf16 high + low parts times the quants."""
    dq, qq = _q8_parts(q[0])                    # (Nh, n_q, 4), (Nh, n_q, D)
    dk, kq = _q8_parts(k[0, 0])                 # (n_kv, 4), (n_kv, D)
    dv, vq = _q8_parts(v[0, 0])
    Nh, n_q, D = qq.shape
    n_kv = kq.shape[0]
    y = np.empty((1, n_q, Nh, D), F)
    for h in range(Nh):
        for iq in range(n_q):
            m, l, o = F(-np.inf), F(0), np.zeros(D, F)
            for t0 in range(0, n_kv, tile):
                kk = slice(t0, min(n_kv, t0 + tile))
                dots = [(kq[kk, 32 * j:32 * j + 32] @ qq[h, iq, 32 * j:32 * j + 32]).astype(F) for j in range(4)]
                w = [(dk[kk, j] * dq[h, iq, j]).astype(F) for j in range(4)]
                sa = (w[1] * dots[1] + (w[0] * dots[0]).astype(F)).astype(F)
                sb = (w[3] * dots[3] + (w[2] * dots[2]).astype(F)).astype(F)
                s = (sa + sb).astype(F)
                mv = mask[0, 0, iq, kk] if mask is not None else np.zeros_like(s)
                x = np.where(mv == -np.inf, F(-np.inf), F(F(s * F(scale)) + mv)).astype(F)
                mn = F(max(m, x.max()))
                if mn == -np.inf:
                    continue
                alpha = F(np.exp(F(m - mn)))
                p = np.exp((x - mn).astype(F)).astype(F)
                m = mn
                l = F(l * alpha)
                o = (o * alpha).astype(F)
                for j in range(p.size):
                    l = F(l + p[j])
                    for bk in range(4):
                        pp = F(p[j] * dv[kk.start + j, bk])
                        hi = orc.bf16_to_f32(orc.f32_to_bf16(np.array([pp], F)))[0]
                        lo = orc.bf16_to_f32(orc.f32_to_bf16(np.array([F(pp - hi)], F)))[0]
                        cols = slice(32 * bk, 32 * bk + 32)
                        o[cols] = (o[cols] + (F(hi) + F(lo)) * vq[kk.start + j, cols]).astype(F)
            y[0, iq, h] = (o * F(F(1) / l)).astype(F)
    return y


def test_emulated_q8_0_decode_kernel_within_bound():
    """The Q8_0 decode kernel's arithmetic (one query position, 4 heads of one KV
    head, scores of several magnitudes) stays inside the q8_0 matrix-core bound,
    which it uses visibly."""
    D, n_kv = 128, 300
    r = np.random.default_rng(9)
    for qscale in (1.0, 6.0):
        q = (r.standard_normal((1, 4, 1, D)) * qscale).astype(F)
        kx = r.standard_normal((1, 1, n_kv, D)).astype(F)
        vx = r.standard_normal((1, 1, n_kv, D)).astype(F)
        m = np.zeros((1, 1, 1, n_kv), F)
        m[..., 250:] = -np.inf
        kf = orc.dequantize_q8_0(orc.quantize_q8_0(kx.reshape(-1, D), "x86")).reshape(kx.shape)
        vf = orc.dequantize_q8_0(orc.quantize_q8_0(vx.reshape(-1, D), "x86")).reshape(vx.shape)
        scale = 1.0 / np.sqrt(D)
        ref = orc.flash_attn_ext(q, kf, vf, m, scale, "q8_0")
        bound = fa_bound(q, kf, vf, m, scale, "q8_0", mfma=True)
        y = _emulate_q8_dec(q, kx, vx, m, scale)
        err = np.abs(y.astype(np.float64) - ref)
        assert np.all(err <= bound), (err / bound).max()
        assert (err / bound).max() > 1e-3


def _bf16(x):
    return orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(x, F)))


def _f16(x):
    return orc.f16_to_f32(orc.f32_to_f16(np.asarray(x, F)))


def _emulate_q8_prefill(q, k, v, mask, scale, tile=64):
    """The Q8_0 matrix-core prefill kernel's arithmetic: q and K as Q8_0 (k holds
    the float rows the quantizer sees), exact int block dots scaled by a chain
    s = fma(d_k d_q, dot, s) in block order; V' = q d_v held as a bf16 high part
    and an fp16 low part; p.V' as (P_hi + P_lo) V_h + RN_fp16(p) V_l."""
    dq, qq = _q8_parts(q[0])
    dk, kq = _q8_parts(k[0, 0])
    dv, vq = _q8_parts(v[0, 0])
    Nh, n_q, D = qq.shape
    n_kv = kq.shape[0]
    vp = (vq * np.repeat(dv, 32, axis=-1)).astype(F)
    vh = _bf16(vp)
    vl = _f16(vp - vh)
    y = np.empty((1, n_q, Nh, D), F)
    for h in range(Nh):
        for iq in range(n_q):
            m, l, o = F(-np.inf), F(0), np.zeros(D, F)
            for t0 in range(0, n_kv, tile):
                kk = slice(t0, min(n_kv, t0 + tile))
                s = None
                for j in range(4):
                    dot = (kq[kk, 32 * j:32 * j + 32] @ qq[h, iq, 32 * j:32 * j + 32]).astype(np.float64)
                    w = (dk[kk, j] * dq[h, iq, j]).astype(np.float64)
                    s = (w * dot).astype(F) if s is None else (w * dot + s).astype(F)
                mv = mask[0, 0, iq, kk] if mask is not None else np.zeros_like(s)
                x = np.where(mv == -np.inf, F(-np.inf), F(F(s * F(scale)) + mv)).astype(F)
                mn = F(max(m, x.max()))
                if mn == -np.inf:
                    continue
                alpha = F(np.exp(F(m - mn)))
                p = np.exp((x - mn).astype(F)).astype(F)
                ph = _bf16(p)
                pl = _bf16(p - ph)
                pf = _f16(p)
                m = mn
                l = F(l * alpha)
                o = (o * alpha).astype(F)
                for j in range(p.size):
                    l = F(l + p[j])
                    o = (o + ph[j] * vh[kk.start + j]).astype(F)
                    o = (o + pl[j] * vh[kk.start + j]).astype(F)
                    o = (o + pf[j] * vl[kk.start + j]).astype(F)
            y[0, iq, h] = (o * F(F(1) / l)).astype(F)
    return y


def test_emulated_q8_0_prefill_kernel_within_bound():
    """The Q8_0 prefill kernel's arithmetic (several query positions and heads of
    one KV head, a causal-style mask, scores of several magnitudes) stays inside
    the q8_0 prefill bound, which it uses visibly."""
    D, n_kv, n_q = 128, 200, 3
    r = np.random.default_rng(11)
    worst = 0.0
    for qscale in (1.0, 6.0):
        q = (r.standard_normal((1, 2, n_q, D)) * qscale).astype(F)
        kx = r.standard_normal((1, 1, n_kv, D)).astype(F)
        vx = r.standard_normal((1, 1, n_kv, D)).astype(F)
        m = np.zeros((1, 1, n_q, n_kv), F)
        for i in range(n_q):
            m[0, 0, i, 150 + 20 * i:] = -np.inf
        kf = orc.dequantize_q8_0(orc.quantize_q8_0(kx.reshape(-1, D), "x86")).reshape(kx.shape)
        vf = orc.dequantize_q8_0(orc.quantize_q8_0(vx.reshape(-1, D), "x86")).reshape(vx.shape)
        scale = 1.0 / np.sqrt(D)
        ref = orc.flash_attn_ext(q, kf, vf, m, scale, "q8_0")
        bound = fa_bound(q, kf, vf, m, scale, "q8_0", mfma="prefill")
        y = _emulate_q8_prefill(q, kx, vx, m, scale)
        err = np.abs(y.astype(np.float64) - ref)
        assert np.all(err <= bound), (err / bound).max()
        worst = max(worst, float((err / bound).max()))
    assert worst > 1e-3


def test_q8_0_v_high_low_parts_hold_every_value_exactly():
    """V' = q d for every int8 q and every finite fp16 d (all 31744 non-negative
    values; the sign is symmetric) is an fp32 value, and a bf16 high part
    RN(V') plus an fp16 low part RN_fp16(V' - RN(V')) hold it exactly, with the
    low part at most 2^-8 |V'| and never overflowing -- the Q8_0 prefill
    kernel's V tile. fma(q + 128, d, -128 d) rounds the exact product, so it
    equals q d."""
    d = orc.f16_to_f32(np.arange(0x7C00, dtype=np.uint16))            # +0 .. 65504
    qs = np.arange(-128, 128, dtype=np.float64)
    for q in qs:
        v = q * d.astype(np.float64)
        vf = v.astype(F)
        assert np.array_equal(vf.astype(np.float64), v)                 # exact in fp32
        vh = _bf16(vf).astype(np.float64)
        vl = _f16((v - vh).astype(F)).astype(np.float64)
        assert np.array_equal(vh + vl, v)
        assert np.all(np.isfinite(vl))
        assert np.all(np.abs(vl) <= 2.0 ** -8 * np.abs(v))


def test_bf16_split_error_reaches_2_to_minus_17():
    """The bf16 high + low split of an fp32 p keeps p within 2^-17 p, and that
    figure is reached: p = 1 + 2^-9 + 2^-17 rounds to 1 + 2^-9 (a tie of the low
    part, to even)."""
    p = np.array([1 + 2.0 ** -9 + 2.0 ** -17], F)
    hi = _bf16(p)
    lo = _bf16((p - hi).astype(F))
    assert float(p[0]) - (float(hi[0]) + float(lo[0])) == 2.0 ** -17
    r = np.random.default_rng(2)
    x = (r.random(1 << 20) * 2.0 ** r.integers(-20, 9, 1 << 20)).astype(F)
    hi = _bf16(x)
    lo = _bf16((x - hi).astype(F))
    err = np.abs(x.astype(np.float64) - hi - lo)
    assert np.all(err <= 2.0 ** -17 * x)


def _case(seed, n_kv, D, qscale, kt):
    r = np.random.default_rng(seed)
    q = (r.standard_normal((1, 2, 3, D)) * qscale).astype(F)
    k = r.standard_normal((1, 1, n_kv, D)).astype(F)
    v = r.standard_normal((1, 1, n_kv, D)).astype(F)
    if kt == "f16":
        k, v = orc.f16_to_f32(orc.f32_to_f16(k)), orc.f16_to_f32(orc.f32_to_f16(v))
    elif kt == "bf16":
        k, v = orc.bf16_to_f32(orc.f32_to_bf16(k)), orc.bf16_to_f32(orc.f32_to_bf16(v))
    m = np.zeros((1, 1, 3, n_kv), F)
    m[0, 0, 1, ::3] = -np.inf
    return q, k, v, m


@pytest.mark.parametrize("kt,mfma", [("f16", False), ("bf16", False), ("f32", False), ("f16", True),
                                     ("bf16", True)])
@pytest.mark.parametrize("n_kv,qscale", [(200, 1.0), (700, 4.0)])
def test_emulated_kernels_within_bound(kt, mfma, n_kv, qscale):
    D = 64
    q, k, v, m = _case(n_kv + D, n_kv, D, qscale, kt)
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn_ext(q, k, v, m, scale, kt)
    bound = fa_bound(q, k, v, m, scale, kt, mfma)
    y = _emulate(q, k, v, m, scale, kt, mfma=mfma, tile=64 if mfma else 32)
    err = np.abs(y.astype(np.float64) - ref)
    assert np.all(err <= bound), (err / bound).max()
    # not vacuous: the emulation's actual error is a visible fraction of the bound
    assert (err / bound).max() > 1e-3


def test_bound_catches_a_dropped_rescale():
    """With the running max's rescale dropped, early tiles keep too much weight:
    the result leaves the bound."""
    D, n_kv = 64, 400
    q, k, v, m = _case(3, n_kv, D, 4.0, "f16")
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn_ext(q, k, v, m, scale, "f16")
    y = _emulate(q, k, v, m, scale, "f16", drop_rescale=True)
    assert np.any(np.abs(y - ref) > fa_bound(q, k, v, m, scale, "f16"))


def test_bound_catches_one_wrong_key_weight():
    """One key's weight off by 1 % (a mask of ln 1.01 on it): the result leaves
    the bound of the unperturbed problem."""
    D, n_kv = 128, 64
    q, k, v, _ = _case(4, n_kv, D, 1.0, "f32")
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn_ext(q, k, v, None, scale, "f32")
    bound = fa_bound(q, k, v, None, scale, "f32")
    m = np.zeros((1, 1, 3, n_kv), F)
    m[..., 5] = np.log(1.01)
    y = orc.flash_attn_ext(q, k, v, m, scale, "f32")
    assert np.any(np.abs(y - ref) > bound)
