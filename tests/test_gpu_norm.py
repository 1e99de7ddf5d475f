"""GPU parity: RMSNorm (+w) and RMSNorm*w -> AdaLN modulate vs the oracle.

fp32: <= 1e-5 relative and, since the kernels sum float squares in double
like ggml-cpu, >= 99.9% of outputs bit-identical (a different summation order
can flip the final float rounding of the mean in rare rows).
bf16: within 1 ulp of the oracle's RNE-rounded fp32 chain. The kernels sum
bf16 squares in fp32 (the oracle in double); the two sums differ by ~2^-18
relative, far inside half a bf16 ulp.
"""
import numpy as np
import pytest
from helpers import assert_bf16_ulp, assert_f32_close, frac_bitexact, randn, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops

pytestmark = pytest.mark.gpu
EPS = 1e-6

SHAPES = [(512, 1024), (97, 2048), (33, 2560), (7, 3000), (5, 96), (300, 128), (40, 64), (11, 256), (3, 4096)]


def _ref(x, w, eps, bf16):
    fn = (lambda a: orc.rms_norm_mul(a, w, eps)) if w is not None else (lambda a: orc.rms_norm(a, eps))
    return orc.bf16_chain(fn, x) if bf16 else fn(x)


@pytest.mark.parametrize("rows,n", SHAPES)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("with_w", [False, True])
def test_rms_norm(dev, rows, n, dt, with_w):
    print(f"rms_norm rows={rows} n={n} {dt} w={with_w}", flush=True)
    x = randn((rows, n), seed=n + rows)
    w = randn((n,), seed=7, scale=0.1, mean=1.0) if with_w else None
    wd = to_dev(w, dev) if with_w else None
    if dt == "bf16":
        xb = orc.f32_to_bf16(x)
        y = ops.rms_norm(to_dev(xb, dev, bf16=True), EPS, w=wd)
        assert_bf16_ulp(to_np(y), _ref(xb, w, EPS, True))
    else:
        y = to_np(ops.rms_norm(to_dev(x, dev), EPS, w=wd))
        ref = _ref(x, w, EPS, False)
        assert_f32_close(y, ref)
        assert frac_bitexact(y, ref) >= 0.999


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rms_norm_strided_rows(dev, dt):
    """Rows of a wider buffer (ggml view with nb1 > ne0*es) and a 4-D view."""
    n, rows, pad = 2048, 24, 512
    big = randn((rows, n + pad), seed=3)
    w = randn((n,), seed=4, scale=0.1, mean=1.0)
    if dt == "bf16":
        bigb = orc.f32_to_bf16(big)
        xd = to_dev(bigb, dev, bf16=True)[:, pad:]
        y = ops.rms_norm(xd, EPS, w=to_dev(w, dev))
        assert_bf16_ulp(to_np(y), _ref(bigb[:, pad:], w, EPS, True))
    else:
        xd = to_dev(big, dev)[:, pad:]
        y = ops.rms_norm(xd, EPS, w=to_dev(w, dev))
        assert_f32_close(to_np(y), _ref(big[:, pad:], w, EPS, False))
    # 4-D [n, 3, 4, 2] view whose rows are strided in every dim
    x4 = to_dev(randn((2, 4, 6, n), seed=5), dev)[:, :, ::2, :]
    y4 = ops.rms_norm(x4, EPS)
    assert_f32_close(to_np(y4), orc.rms_norm(to_np(x4), EPS))


@pytest.mark.parametrize("n", [64, 128, 256])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_rms_norm_head_rows(dev, n, dt):
    """Head-sized rows (the per-head Q/K norm) of row-uniform views take the
    whole-row kernel: 70001 contiguous rows (several chunks per wave, a ragged
    last chunk) with w, then rows of a wider buffer (nb1 > ne0*es) without w,
    then a [n, 5, 7, 3] 4-D view. f16 outputs within 1 f16 ulp of the oracle's
    RNE-rounded fp32 chain, f32 at 1e-5 and >= 99.9 % bit-identical."""
    print(f"rms_norm head rows n={n} {dt}", flush=True)
    f32 = dt == "f32"
    enc = {"bf16": orc.f32_to_bf16, "f16": orc.f32_to_f16}.get(dt)
    dec = {"bf16": orc.bf16_to_f32, "f16": orc.f16_to_f32}.get(dt)

    def dev_of(a):
        return to_dev(a, dev) if f32 else to_dev(a, dev, bf16=dt == "bf16", f16=dt == "f16")

    def check(y, xh, w):
        fn = (lambda a: orc.rms_norm_mul(a, w, EPS)) if w is not None else (lambda a: orc.rms_norm(a, EPS))
        if f32:
            ref = fn(xh)
            assert_f32_close(y, ref)
            assert frac_bitexact(y, ref) >= 0.999
        else:
            assert_bf16_ulp(y, enc(fn(dec(xh))))  # sign-magnitude ordinal: an f16 ulp as well

    w = randn((n,), seed=n, scale=0.1, mean=1.0)
    x = randn((70001, n), seed=n + 1)
    xh = x if f32 else enc(x)
    check(to_np(ops.rms_norm(dev_of(xh), EPS, w=to_dev(w, dev))), xh, w)
    pad = 48
    big = randn((301, n + pad), seed=n + 2)
    bh = big if f32 else enc(big)
    check(to_np(ops.rms_norm(dev_of(bh)[:, pad:], EPS)), np.ascontiguousarray(bh[:, pad:]), None)
    x4 = randn((3, 7, 5, n), seed=n + 3)
    x4h = x4 if f32 else enc(x4)
    check(to_np(ops.rms_norm(dev_of(x4h), EPS, w=to_dev(w, dev))), x4h, w)


def test_rms_norm_unaligned_generic_path(dev):
    """A 4-byte (not 16-byte) aligned view falls back to the scalar path."""
    n, rows = 1024, 9
    buf = randn((rows * n + 1,), seed=8)
    xd = to_dev(buf, dev)[1:].view(rows, n)
    y = ops.rms_norm(xd, EPS)
    ref = orc.rms_norm(buf[1:].reshape(rows, n), EPS)
    assert_f32_close(to_np(y), ref)


def test_rms_norm_bf16_generic_path_matches_fast_path(dev):
    """A BF16 view 2 bytes off 16-byte alignment takes the generic kernel, its
    aligned copy the fast one. Both sum the squares in fp32 (the fast kernels'
    accumulator for 16-bit rows); the orders differ, so the final rounding may
    too: each result within 1 ulp of the oracle and of the other, and almost all
    outputs bit-identical."""
    n, rows = 2048, 37
    xb = orc.f32_to_bf16(randn((rows * n + 1,), seed=21))
    w = randn((n,), seed=22, scale=0.1, mean=1.0)
    wd = to_dev(w, dev)
    un = to_dev(xb, dev, bf16=True)[1:].view(rows, n)
    al = to_dev(np.ascontiguousarray(xb[1:]).reshape(rows, n), dev, bf16=True)
    yg = to_np(ops.rms_norm(un, EPS, w=wd))
    yf = to_np(ops.rms_norm(al, EPS, w=wd))
    ref = _ref(xb[1:].reshape(rows, n), w, EPS, True)
    assert_bf16_ulp(yg, ref)
    assert_bf16_ulp(yf, ref)
    assert_bf16_ulp(yg, yf)
    assert frac_bitexact(yg, yf) >= 0.99


@pytest.mark.parametrize("rows,n", [(600, 2048), (37, 1024), (5, 3000)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rms_norm_modulate(dev, rows, n, dt):
    print(f"rms_norm_modulate rows={rows} n={n} {dt}", flush=True)
    x = randn((rows, n), seed=11)
    w = randn((n,), seed=12, scale=0.1, mean=1.0)
    sc = randn((n,), seed=13, scale=0.1)
    sh = randn((n,), seed=14, scale=0.1)
    args = [to_dev(a, dev) for a in (w, sc, sh)]
    if dt == "bf16":
        xb = orc.f32_to_bf16(x)
        y = ops.rms_norm_modulate(to_dev(xb, dev, bf16=True), *args, EPS)
        ref = orc.bf16_chain(lambda a: orc.rms_norm_modulate(a, w, sc, sh, EPS), xb)
        assert_bf16_ulp(to_np(y), ref)
    else:
        y = to_np(ops.rms_norm_modulate(to_dev(x, dev), *args, EPS))
        ref = orc.rms_norm_modulate(x, w, sc, sh, EPS)
        assert_f32_close(y, ref, row_floor=True)
        assert frac_bitexact(y, ref) >= 0.999


def test_rms_norm_special_rows(dev):
    """All-zero row (scale = 1/sqrt(eps)), tiny and huge magnitudes."""
    n = 1024
    x = np.zeros((4, n), np.float32)
    x[1] = 1e-20
    x[2] = randn((n,), seed=1) * 1e18
    x[3, ::7] = -3.0
    y = to_np(ops.rms_norm(to_dev(x, dev), EPS))
    assert_f32_close(y, orc.rms_norm(x, EPS))


@pytest.mark.parametrize("rows,n", [(600, 2048), (33, 2560), (50, 1024), (7, 3000), (9, 128)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_add_rms_norm_gated_modulate(dev, rows, n, dt):
    """DiT: h1 = h + sa_out * gate_sa; norm_ffn = rms_norm(h1) * w -> AdaLN (dit-graph.h:420, 442-443)."""
    print(f"add_rms_norm gated+mod rows={rows} n={n} {dt}", flush=True)
    bf16 = dt == "bf16"
    h = randn((rows, n), seed=21)
    x = randn((rows, n), seed=22)
    gate, w = randn((n,), seed=23, scale=0.1), randn((n,), seed=24, scale=0.1, mean=1.0)
    sc, sh = randn((n,), seed=25, scale=0.1), randn((n,), seed=26, scale=0.1)
    hh = orc.f32_to_bf16(h) if bf16 else h
    xh = orc.f32_to_bf16(x) if bf16 else x
    vd = [to_dev(v, dev) for v in (gate, w, sc, sh)]
    ys, yn = ops.add_rms_norm(to_dev(hh, dev, bf16=bf16), to_dev(xh, dev, bf16=bf16), EPS, gate=vd[0], w=vd[1],
                              scale=vd[2], shift=vd[3])
    f = orc.bf16_to_f32 if bf16 else (lambda a: a)
    s_ref = orc.gated_add(f(hh), f(xh), gate)
    if bf16:
        s_ref = orc.f32_to_bf16(s_ref)
        assert np.array_equal(to_np(ys), s_ref)
        assert_bf16_ulp(to_np(yn), orc.bf16_chain(lambda a: orc.rms_norm_modulate(a, w, sc, sh, EPS), s_ref))
    else:
        assert np.array_equal(to_np(ys), s_ref)
        ref = orc.rms_norm_modulate(s_ref, w, sc, sh, EPS)
        assert_f32_close(to_np(yn), ref, row_floor=True)
        assert frac_bitexact(to_np(yn), ref) >= 0.999


@pytest.mark.parametrize("n", [2560, 2048, 96])
def test_add_clamp_rms_norm_in_place(dev, n):
    """Qwen3: hidden = clamp(hidden + attn_out); norm2 = rms_norm(hidden) * w (qwen3-lm.h:730-736),
    with y_sum written in place over the residual."""
    rows = 40
    h = randn((rows, n), seed=31)
    h[0, :3] = [7e4, -7e4, 6e4]
    a = randn((rows, n), seed=32)
    w = randn((n,), seed=33, scale=0.1, mean=1.0)
    hd = to_dev(h, dev)
    ys, yn = ops.add_rms_norm(hd, to_dev(a, dev), EPS, w=to_dev(w, dev), clamp=(-65504.0, 65504.0), out_sum=hd)
    s_ref = orc.add_clamp(h, a)
    assert np.array_equal(to_np(hd), s_ref)
    ref = orc.rms_norm_mul(s_ref, w, EPS)
    assert_f32_close(to_np(yn), ref)
    assert frac_bitexact(to_np(yn), ref) >= 0.999
