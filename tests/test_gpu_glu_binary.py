"""GPU parity: SwiGLU (fused / swapped / split) and the elementwise ops
(residual add, add+clamp, gated residual, AdaLN modulate, mul) vs the oracle.

SwiGLU uses the device exp2/rcp with an fma-recovered exponent, so the fp32
bar is relative (<= 1e-5, denominator floored at 1e-30 for the -0/denormal
tail where ggml's expf overflows). The elementwise ops keep ggml's operation
order exactly, so they are checked bit-for-bit.
"""
import numpy as np
import pytest
from helpers import assert_bf16_ulp, assert_f32_close, randn, rng, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,n", [(512, 3072), (8, 9728), (120, 6144), (3, 1000), (5, 12)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_swiglu_fused(dev, rows, n, dt):
    print(f"swiglu rows={rows} n={n} {dt}", flush=True)
    gu = randn((rows, 2 * n), seed=rows + n)
    if dt == "bf16":
        gb = orc.f32_to_bf16(gu)
        y = ops.swiglu(to_dev(gb, dev, bf16=True))
        assert_bf16_ulp(to_np(y), orc.bf16_chain(orc.swiglu, gb))
    else:
        y = ops.swiglu(to_dev(gu, dev))
        assert_f32_close(to_np(y), orc.swiglu(gu))


def test_swiglu_swapped_and_split(dev):
    gu = randn((64, 2 * 1024), seed=3)
    y = ops.swiglu(to_dev(gu, dev), swapped=True)
    assert_f32_close(to_np(y), orc.swiglu(gu, swapped=True))
    g = randn((64, 3072), seed=4)
    u = randn((64, 3072), seed=5)
    y = ops.swiglu_split(to_dev(g, dev), to_dev(u, dev))
    assert_f32_close(to_np(y), orc.swiglu_split(g, u))


def test_swiglu_extreme_gates(dev):
    """Gates across the whole range: overflow of e^-g (-> -0), large g (-> g*u), 0, +-inf, NaN."""
    g = np.concatenate([
        np.linspace(-120, 120, 4096, dtype=np.float32),
        np.array([0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, -88.7, -88.8, -90.0, 3.4e38, -3.4e38], np.float32),
    ])
    g = np.concatenate([g, np.zeros((-g.size) % 8, np.float32)])
    u = randn(g.shape, seed=6)
    y = to_np(ops.swiglu_split(to_dev(g[None], dev), to_dev(u[None], dev)))[0]
    ref = orc.swiglu_split(g[None], u[None])[0]
    assert_f32_close(y, ref)
    g2 = np.array([np.inf, -np.inf, np.nan, 1.0] * 2, np.float32)
    u2 = np.ones(8, np.float32)
    y2 = to_np(ops.swiglu_split(to_dev(g2[None], dev), to_dev(u2[None], dev)))[0]
    r2 = orc.swiglu_split(g2[None], u2[None])[0]
    assert np.array_equal(np.isnan(y2), np.isnan(r2))
    assert np.array_equal(y2[~np.isnan(r2)], r2[~np.isnan(r2)])


def _bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("n", [2048, 2560, 1024, 200])
def test_elementwise_bitexact(dev, dt, n):
    print(f"elementwise n={n} {dt}", flush=True)
    rows = 77
    a = randn((rows, n), seed=1)
    b = randn((rows, n), seed=2)
    vec = randn((n,), seed=3, scale=0.1)
    vec2 = randn((n,), seed=4, scale=0.1)
    bf16 = dt == "bf16"
    ah = orc.f32_to_bf16(a) if bf16 else a
    bh = orc.f32_to_bf16(b) if bf16 else b
    ad, bd = to_dev(ah, dev, bf16=bf16), to_dev(bh, dev, bf16=bf16)
    vd, v2d = to_dev(vec, dev), to_dev(vec2, dev)
    cases = [
        (ops.add(ad, bd), lambda x, y: orc.add(x, y)),
        (ops.add(ad, vd), lambda x, y: orc.add(x, vec)),
        (ops.mul(ad, vd), lambda x, y: orc.mul(x, vec)),
        (ops.mul(ad, bd), lambda x, y: orc.mul(x, y)),
        (ops.gated_add(ad, bd, vd), lambda x, y: orc.gated_add(x, y, vec)),
        (ops.modulate(ad, vd, v2d), lambda x, y: orc.adaln_modulate(x, vec, vec2)),
        (ops.add_clamp(ad, bd, -1.5, 2.0), lambda x, y: orc.add_clamp(x, y, -1.5, 2.0)),
    ]
    for i, (got, fn) in enumerate(cases):
        ref = orc.bf16_chain(fn, ah, bh) if bf16 else fn(a, b)
        assert _bits_equal(to_np(got), ref), f"case {i} differs"


def test_add_clamp_fp16_range_outliers(dev):
    """Residual add + FP16 clamp with 0.1% outliers ~N(0,1000) and +-1e5 injections."""
    rows, n = 64, 2048
    a = randn((rows, n), seed=5)
    b = randn((rows, n), seed=6)
    r = rng(7)
    idx = r.choice(a.size, a.size // 1000, replace=False)
    a.reshape(-1)[idx] = (r.standard_normal(idx.size) * 1000).astype(np.float32)
    a.reshape(-1)[r.choice(a.size, 16, replace=False)] = np.float32(1e5) * np.sign(r.standard_normal(16)).astype(np.float32)
    a.reshape(-1)[3] = np.nan
    y = to_np(ops.add_clamp(to_dev(a, dev), to_dev(b, dev)))
    ref = orc.add_clamp(a, b)
    assert _bits_equal(y, ref)
    assert y.reshape(-1)[3] == 65504.0  # MIN(NaN, hi) -> hi, as the ggml macro does


def test_binary_general_broadcast(dev):
    """ggml_can_repeat broadcasts other than a row vector take the generic path."""
    a = randn((4, 6, 10, 32), seed=8)
    b = randn((1, 6, 1, 32), seed=9)
    y = to_np(ops.add(to_dev(a, dev), to_dev(b, dev)))
    ref = a + b  # one IEEE add per element, same as ggml_add
    assert _bits_equal(y, ref)
    y = to_np(ops.mul(to_dev(a, dev), to_dev(b, dev)))
    assert _bits_equal(y, a * b)


def test_in_place_gated_add(dev):
    n = 2048
    res = randn((33, n), seed=1)
    x = randn((33, n), seed=2)
    g = randn((n,), seed=3, scale=0.1)
    rd = to_dev(res, dev)
    ops.gated_add(rd, to_dev(x, dev), to_dev(g, dev), out=rd)
    assert _bits_equal(to_np(rd), orc.gated_add(res, x, g))


@pytest.mark.parametrize("T", [1, 3])
def test_views_with_packed_inner_rows(dev, T):
    """[D, nkv, T, B] views of a fused QKV buffer (the decode-time V view):
    rows inside a token are packed but tokens sit a whole QKV row apart, so
    row addressing must not treat them as uniformly strided, also when T = 1."""
    B, nh, nkv, D = 4, 4, 2, 128
    W = (nh + 2 * nkv) * D
    qkv = randn((B, T, W), seed=21)
    qkv[0, 0, (nh + nkv) * D + 5] = 7e4
    qd = to_dev(qkv, dev)
    vd = qd[:, :, (nh + nkv) * D:].unflatten(2, (nkv, D))
    v = qkv[:, :, (nh + nkv) * D:].reshape(B, T, nkv, D)
    other = randn((B, T, nkv, D), seed=22)
    y = to_np(ops.add(vd, to_dev(other, dev)))
    assert _bits_equal(y, v + other)
    y = to_np(ops.rms_norm(vd, 1e-6))
    assert_f32_close(y, orc.rms_norm(v, 1e-6))
    ops.clamp(vd, -65504.0, 65504.0, out=vd)  # in place, as the layer driver does
    got = to_np(qd)
    ref = qkv.copy()
    ref[:, :, (nh + nkv) * D:] = orc.clamp(qkv[:, :, (nh + nkv) * D:], -65504.0, 65504.0)
    assert _bits_equal(got, ref)
