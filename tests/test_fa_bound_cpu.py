"""The flash-attention error bound (tests/fa_bound.py) against fp32 emulations
of the kernels' arithmetic on the CPU: the split-key path (sequential fp32 dot
products, tile-wise running max with rescales, fp32 accumulation of o and l)
and the matrix-core path (P as high + low 16-bit parts in the p.V product, l
from the fp32 p). Each emulation must stay inside the bound, including at
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
