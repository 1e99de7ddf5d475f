"""Pins the CPU oracle before the tests trust it as their reference (CPU only).

ggml is absent from the reference checkout and the reference's tests hold no
golden vectors for these ops, so each oracle function is pinned here by
checks that do not restate its own formula: numpy's independent float16
conversion, float64 mathematics, brute force over small domains, exact
invariances (power-of-two scaling, position 0, pair norms) and closed forms.
Each group names the mistake it is built to catch.
"""
import numpy as np
import pytest

from helpers import randn, rng
from oracle import oracle as orc


def _u32(x):
    return np.asarray(x, np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# number formats
# ---------------------------------------------------------------------------
def _all_f32_sample(n=1 << 22, seed=0):
    """Random bit patterns plus every fp16/bf16 rounding boundary class."""
    r = rng(seed)
    bits = r.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    return bits.view(np.float32)


def test_fp16_conversions_match_numpy():
    """Catches: truncation instead of RNE, wrong subnormal/overflow thresholds."""
    h = np.arange(1 << 16, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = orc.f16_to_f32(h)
    fin = ~np.isnan(ref)
    assert np.array_equal(_u32(got[fin]), _u32(ref[fin]))
    assert np.all(np.isnan(got[~fin]))
    x = _all_f32_sample()
    # every halfway point between adjacent fp16 values, and its neighbours
    with np.errstate(invalid="ignore"):
        mids = ((h[:-1].view(np.float16).astype(np.float64) + h[1:].view(np.float16).astype(np.float64)) / 2)
    mids = mids[np.isfinite(mids)].astype(np.float32)
    x = np.concatenate([x, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                        np.float32([65504, 65519.996, 65520, -65520, 2 ** -25, 2 ** -24, 3 * 2 ** -26])])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = orc.f32_to_f16(x)
    fin = ~np.isnan(x)
    assert np.array_equal(got[fin], ref[fin])
    assert np.all(np.isnan(got[~fin].view(np.float16)))


def test_bf16_rne_against_nearest_neighbour_search():
    """Catches: truncation, ties away from zero, NaN turned into inf."""
    x = np.concatenate([_all_f32_sample(seed=1),
                        # exact ties: low 16 bits = 0x8000 with odd and even kept lsb
                        (np.arange(0, 1 << 16, 7, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    u = _u32(x)
    lo = (u & 0xFFFF0000).view(np.float32)             # truncation toward zero
    hi = ((u & 0xFFFF0000) + 0x10000).astype(np.uint32).view(np.float32)  # next bf16 away from zero
    with np.errstate(invalid="ignore", over="ignore"):
        xd, lod, hid = (np.asarray(v, np.float64) for v in (x, lo, hi))
        dlo, dhi = np.abs(xd - lod), np.abs(hid - xd)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (((u >> 16) & 1) == 1))
    ref = np.where(pick_hi, (u + 0x10000) >> 16, u >> 16).astype(np.uint16)
    got = orc.f32_to_bf16(x)
    fin = np.isfinite(x) & np.isfinite(hi)
    assert np.array_equal(got[fin], ref[fin])
    nan = np.isnan(x)
    assert np.all(np.isnan(orc.bf16_to_f32(got[nan])))
    back = orc.bf16_to_f32(got[fin])
    assert np.array_equal(_u32(back), (got[fin].astype(np.uint32) << 16))


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
def test_rms_norm_against_float64_and_closed_forms():
    """Catches: dropped eps, mean over n-1, missing sqrt, float (not double) sum drift."""
    for n, eps in ((2048, 1e-6), (128, 1e-6), (1000, 1e-5), (7, 0.1)):
        x = randn((64, n), seed=n, scale=3.0)
        y = orc.rms_norm(x, eps)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + eps)
        assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) < 4e-7
    # constant row: y = c / sqrt(c^2 + eps) exactly up to fp32 rounding
    c = np.full((1, 1024), 0.25, np.float32)
    assert np.allclose(orc.rms_norm(c, 1e-2), 0.25 / np.sqrt(0.0625 + 1e-2), rtol=2e-7, atol=0)


def test_rms_norm_power_of_two_scaling_is_bit_exact():
    """With eps = 0, x*2^k scales every float square, the double sum, the
    mean and sqrtf by exact powers of two, so the output is bit-identical.
    Catches: an inexact reduction order change that still looks close."""
    x = randn((32, 2048), seed=3)
    y0 = orc.rms_norm(x, 0.0)
    for k in (-20, -3, 5, 30):
        assert np.array_equal(_u32(orc.rms_norm(x * np.float32(2.0 ** k), 0.0)), _u32(y0))


def test_rms_norm_long_double_brute_force_tiny_rows():
    """Rows of 1..8 elements against exact rational arithmetic of the same steps."""
    from fractions import Fraction as Fr
    r = rng(5)
    for n in range(1, 9):
        x = (r.standard_normal((20, n)) * 10).astype(np.float32)
        y = orc.rms_norm(x, 1e-6)
        for i in range(20):
            ms = sum(Fr(float(np.float32(v) * np.float32(v))) for v in x[i]) / n   # float squares, exact sum
            mean = np.float32(float(ms))
            scale = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(1e-6)))
            assert np.array_equal(_u32(y[i]), _u32(x[i] * scale))


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------
def test_elementwise_ieee_and_ggml_clamp_semantics():
    """add/mul are single IEEE fp32 operations; ggml_clamp is MAX(MIN(x,hi),lo)
    with the comparison macros, so NaN maps to hi. Catches: fused or reordered
    chains, fmaxf/fminf NaN handling."""
    a, b = randn((8, 64), seed=1), randn((8, 64), seed=2)
    v = randn((64,), seed=3)
    assert np.array_equal(_u32(orc.add(a, b)), _u32(a + b))
    assert np.array_equal(_u32(orc.mul(a, v)), _u32(a * v))
    assert np.array_equal(_u32(orc.gated_add(a, b, v)), _u32(a + b * v))
    assert np.array_equal(_u32(orc.adaln_modulate(a, v, b[0])), _u32(a * (v + np.float32(1)) + b[0]))
    x = np.float32([np.nan, np.inf, -np.inf, 7e4, -7e4, 1.0, -0.0])
    y = orc.clamp(x, -65504.0, 65504.0)
    assert y[0] == 65504.0 and y[1] == 65504.0 and y[2] == -65504.0 and y[3] == 65504.0 and y[4] == -65504.0
    assert y[5] == 1.0 and np.signbit(y[6])


def test_scale_is_the_correctly_rounded_product():
    """ggml_scale: y = x * s rounded once. The product of two floats is exact in
    double (24 + 24 significand bits), so rounding the double product to float
    once is the correctly rounded fp32 product. Catches: a reciprocal-based or
    double-rounded scale, a dropped sign, x + s."""
    r = np.random.default_rng(9)
    x = (r.standard_normal(4096) * np.exp2(r.integers(-140, 120, 4096))).astype(np.float32)
    x[:6] = [0.0, -0.0, np.inf, -np.inf, 1.17549435e-38, 3.4e38]
    for s in (1000.0, -0.37, 3.0, 2.0 ** -30, 1e30):
        want = (x.astype(np.float64) * np.float64(np.float32(s))).astype(np.float32)
        assert np.array_equal(_u32(orc.scale(x, s)), _u32(want)), s
    y = orc.scale(np.float32([np.nan, 1.0]), 2.0)
    assert np.isnan(y[0]) and y[1] == 2.0


# ---------------------------------------------------------------------------
# NEOX rope
# ---------------------------------------------------------------------------
def _angles_from_unit_pairs(pos, D, base, **kw):
    """Rotate (1, 0) pairs; the outputs are (cos, sin) of the oracle's angles."""
    x = np.zeros((len(pos), 1, D), np.float32)
    x[:, :, :D // 2] = 1.0
    y = orc.rope_neox(x, np.asarray(pos, np.int32), D, base, **kw)
    return y[:, 0, :D // 2].astype(np.float64), y[:, 0, D // 2:].astype(np.float64)


def test_rope_position_zero_identity_and_pair_norms():
    """Catches: swapped halves, wrong sign of the sin term, non-rotation."""
    x = randn((3, 16, 128), seed=7)
    y = orc.rope_neox(x, np.int32([0, 5, 4000]), 128, 1e6)
    assert np.array_equal(_u32(y[0]), _u32(x[0]))
    n_in = np.hypot(x[..., :64].astype(np.float64), x[..., 64:])
    n_out = np.hypot(y[..., :64].astype(np.float64), y[..., 64:])
    assert np.max(np.abs(n_out - n_in) / np.maximum(n_in, 1e-6)) < 5e-7
    # y_i = x_i c - x_{i+h} s with s = sin(+theta): (0, 1) at p = 1, pair 0 -> (-sin 1, cos 1)
    e = np.zeros((1, 1, 128), np.float32)
    e[..., 64] = 1.0
    y = orc.rope_neox(e, np.int32([1]), 128, 1e6)
    assert abs(y[0, 0, 0] + np.sin(1.0)) < 1e-7 and abs(y[0, 0, 64] - np.cos(1.0)) < 1e-7


def test_rope_angles_follow_float_chain_not_powf():
    """ggml builds theta_i by repeated fp32 multiplication. At p = 8191 that
    chain and p * powf(base, -2i/D) differ by far more than sin/cos error, so
    an oracle using the closed form fails. Also pins theta_scale = powf(base, -2/D)."""
    D, base = 128, 1e6
    pos = np.int32([8191, 511, 3])
    c, s = _angles_from_unit_pairs(pos, D, base)
    ts = np.float32(base) ** np.float32(-2.0 / D)
    assert orc.rope_theta_scale(base, D) == ts
    chain = np.empty((len(pos), D // 2), np.float32)
    th = pos.astype(np.float32)
    for i in range(D // 2):
        chain[:, i] = th
        th = (th * ts).astype(np.float32)
    assert np.max(np.abs(c - np.cos(chain.astype(np.float64)))) < 2e-7
    assert np.max(np.abs(s - np.sin(chain.astype(np.float64)))) < 2e-7
    exact = pos[:, None].astype(np.float64) * np.float64(base) ** (-2.0 * np.arange(D // 2) / D)
    drift = np.abs(np.angle(np.exp(1j * (chain.astype(np.float64) - exact))))
    assert drift[0].max() > 1e-4          # the chain is visibly not the closed form at p = 8191 (3.4e-4 rad)
    assert drift[2].max() < 1e-5          # and agrees with it at small positions
    assert np.max(np.abs(c[0] - np.cos(exact[0]))) > 1e-4   # so a closed-form oracle would fail the 2e-7 bar


def test_rope_partial_dims_freq_scale_attn_factor():
    """Dims >= n_dims are copied; attn_factor = 2 doubles cos/sin exactly;
    freq_scale multiplies the angle. Catches: rotating the tail, ignoring scales."""
    x = randn((4, 8, 96), seed=9)
    pos = np.int32([0, 1, 100, 2000])
    y = orc.rope_neox(x, pos, 64, 1e4)
    assert np.array_equal(_u32(y[..., 64:]), _u32(x[..., 64:]))
    c1, s1 = _angles_from_unit_pairs(pos, 64, 1e4)
    c2, s2 = _angles_from_unit_pairs(pos, 64, 1e4, attn_factor=2.0)
    assert np.array_equal(c2, 2 * c1) and np.array_equal(s2, 2 * s1)
    c3, _ = _angles_from_unit_pairs(pos, 64, 1e4, freq_scale=0.5)
    ang = np.float32(0.5) * np.float32(100.0)
    assert abs(c3[2, 0] - np.cos(np.float64(ang))) < 1e-7


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def test_swiglu_against_float64_and_special_values():
    """Catches: sigmoid(x) instead of silu, halves swapped, expf(x) sign flip."""
    g = np.concatenate([randn((4096,), seed=1, scale=6.0), np.float32([0.0, -0.0, 100.0, -100.0, -90.0, 88.0,
                                                                       np.inf, -np.inf, np.nan])])
    u = randn(g.shape, seed=2)
    y = orc.swiglu_split(g, u)
    gd = g.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = gd / (1.0 + np.exp(-gd)) * u
    m = np.isfinite(g) & (np.abs(g) < 80)
    assert np.max(np.abs(y[m] - ref[m]) / np.maximum(np.abs(ref[m]), 1e-30)) < 4e-7
    k = g.size - 9
    assert y[k] == 0 and y[k + 2] == np.float32(100.0) * u[k + 2]
    for i in (k + 3, k + 4):      # expf(-g) overflows to inf for g < -88.7: g/inf = -0, times u
        assert y[i] == 0 and np.signbit(y[i]) != np.signbit(u[i])
    assert y[k + 5] == np.float32(88.0) * u[k + 5]                           # 1 + expf(-88) rounds to 1
    assert y[k + 6] == np.float32(np.inf) * u[k + 6]                         # inf / (1 + 0)
    assert np.isnan(y[k + 7]) and np.isnan(y[k + 8])                         # -inf / inf, NaN
    gu = np.concatenate([g[None, :64], u[None, :64]], axis=1)
    assert np.array_equal(_u32(orc.swiglu(gu)), _u32(orc.swiglu_split(g[None, :64], u[None, :64])))
    assert np.array_equal(_u32(orc.swiglu(gu, swapped=True)), _u32(orc.swiglu_split(u[None, :64], g[None, :64])))


# ---------------------------------------------------------------------------
# Q8_0
# ---------------------------------------------------------------------------
def _q8_blocks(q_int8, d_f16_bits):
    nb = len(d_f16_bits)
    raw = np.zeros((nb, 34), np.uint8)
    raw[:, :2] = np.asarray(d_f16_bits, np.uint16).reshape(-1, 1).view(np.uint8)
    raw[:, 2:] = np.asarray(q_int8, np.int8).reshape(nb, 32).view(np.uint8)
    return raw.reshape(-1)


def test_q8_0_dequant_brute_force_exact():
    """All 256 int8 values x fp16 scales (0, subnormal, normal, max): the
    product is exact in fp32. Catches: uint8 read of the quants, scale byte order."""
    scales = np.concatenate([np.uint16([0, 1, 0x3FF, 0x400, 0x3C00, 0x7BFF, 0x8001, 0xBC00]),
                             rng(3).integers(0, 0x7C00, 56).astype(np.uint16)])
    q = np.tile(np.arange(-128, 128, dtype=np.int16).astype(np.int8), 8).reshape(8, 256)
    for d in scales:
        raw = _q8_blocks(q.reshape(-1), np.full(q.size // 32, d, np.uint16))
        y = orc.dequantize_q8_0(raw)
        ref = q.reshape(-1).astype(np.float64) * np.float64(np.uint16(d).view(np.float16))
        assert np.array_equal(y.astype(np.float64), ref)


def test_q8_0_quantize_invariants_both_variants():
    """|q| <= 127, the block's largest |x| maps to +-127, |x - q d| <= d/2
    (+ rounding slack), zero blocks give d = 0, q = 0; dequant of the result
    recovers q*d exactly. Catches: scale from mean instead of amax, clipping at
    128, truncating rounding."""
    x = randn((64, 256), seed=11)
    x[3, :32] = 0.0
    for variant in ("ref", "x86"):
        raw = orc.quantize_q8_0(x, variant).reshape(64, 8, 34)
        d = raw[..., :2].copy().view(np.uint16).reshape(64, 8).view(np.float16).astype(np.float32)
        q = raw[..., 2:].view(np.int8).astype(np.int32)
        assert np.all(np.abs(q) <= 127)
        xb = x.reshape(64, 8, 32)
        am = np.argmax(np.abs(xb), axis=-1)
        top = np.take_along_axis(q, am[..., None], -1)[..., 0]
        nz = d != 0
        assert np.all(np.abs(top[nz]) == 127)
        # half a step, plus the fp16 rounding of d seen through |q| <= 127 (127 * 2^-11 d)
        err = np.abs(xb - q * d[..., None])
        assert np.all(err <= d[..., None] * (0.5 + 127 * 2.0 ** -11) + 1e-7)
        assert np.mean(err) < 0.3 * np.mean(d)   # truncation would average ~d/2
        assert d[3, 0] == 0 and np.all(q[3, 0] == 0)
        back = orc.dequantize_q8_0(raw.reshape(64, -1))
        assert np.array_equal(back.reshape(64, 8, 32), (q * d[..., None]).astype(np.float32))


def test_q8_0_variants_separate_on_ties_and_reciprocals():
    """REF rounds half away from zero with id = 1/(amax/127); X86 rounds half
    to even with id = 127/amax. Blocks built so x*id is exactly k + 0.5 tell
    them apart; so do amax values where the two ids differ in fp32."""
    # amax = 127 -> d = 1, id = 1 in both; x = k + 0.5 are exact ties
    blk = np.zeros(32, np.float32)
    blk[0] = 127.0
    blk[1:9] = np.float32([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5])
    qr = orc.quantize_q8_0(blk[None], "ref")[0, 2:].view(np.int8)
    qx = orc.quantize_q8_0(blk[None], "x86")[0, 2:].view(np.int8)
    assert list(qr[1:9]) == [1, 2, 3, -1, -2, -3, 127, -127]
    assert list(qx[1:9]) == [0, 2, 2, 0, -2, -2, 126, -126]
    # amax where 127/amax != 1/(amax/127) in fp32: the quants of some x differ
    r = rng(13)
    found = 0
    for amax in r.uniform(0.01, 10, 4000).astype(np.float32):
        id_x86 = np.float32(127) / amax
        id_ref = np.float32(1) / (amax / np.float32(127))
        if id_x86 == id_ref:
            continue
        b = np.float32(r.uniform(-1, 1, 32)) * amax
        b[0] = amax
        # put one element on the rounding boundary of one variant
        k = np.float32(37.5)
        b[1] = np.float32(k / id_x86)
        if np.float32(b[1] * id_x86) == k and np.float32(b[1] * id_ref) != k:
            a1 = orc.quantize_q8_0(b[None], "ref")[0, 3].view(np.int8)
            a2 = orc.quantize_q8_0(b[None], "x86")[0, 3].view(np.int8)
            found += int(a1 != a2)
    assert found > 0


def test_get_rows_plain_types_and_bounds():
    tab = randn((50, 64), seed=4)
    ids = np.int32([0, 49, 7, 7, 13])
    assert np.array_equal(orc.get_rows(tab, orc.F32, 64, ids), tab[ids])
    h = tab.astype(np.float16)
    assert np.array_equal(orc.get_rows(h.view(np.uint16), orc.F16, 64, ids), h[ids].astype(np.float32))
    bf = orc.f32_to_bf16(tab)
    assert np.array_equal(orc.get_rows(bf, orc.BF16, 64, ids), orc.bf16_to_f32(bf)[ids])
    with pytest.raises(IndexError):
        orc.get_rows(tab, orc.F32, 64, np.int32([50]))


# ---------------------------------------------------------------------------
# timestep embedding
# ---------------------------------------------------------------------------
def test_timestep_embedding_against_float64():
    """out[j] = cos(t f_j), out[j + half] = sin(t f_j), f_j = exp(-ln(P) j / half).
    The oracle evaluates f_j in fp32: the exponent -ln(P) j / half carries
    ~2^-23 relative error, which expf turns into ln(P) * 2^-23 relative error
    of f_j, and t*f_j adds one more rounding; so the bound is
    (1 + ln P) 2^-23 |t f_j| + 1e-7. Catches: cos/sin halves swapped,
    j/(half-1), log2, max_period ignored."""
    t = np.float32([0.0, 0.37, 1.0, 250.0, 999.0])
    y = orc.timestep_embedding(t, 256, 10000)
    half = 128
    f = np.exp(-np.log(10000.0) * np.arange(half) / half)
    arg = t[:, None].astype(np.float64) * f
    ref = np.concatenate([np.cos(arg), np.sin(arg)], axis=1)
    bound = np.concatenate([np.abs(arg), np.abs(arg)], axis=1) * (1 + np.log(10000.0)) * 2.0 ** -23 + 1e-7
    assert np.all(np.abs(y - ref) <= bound)
    assert np.array_equal(y[0, :half], np.ones(half, np.float32)) and np.all(y[0, half:] == 0)
