"""Pinning the flash-attention oracle (orc_flash_attn_ext) without ggml.

Each check is fixed by the mathematics, not by restating the oracle's loop,
and a plausible mistake fails at least one of them:
  one key -> v exactly; equal scores (q = 0, or scale = 0) -> mean of v;
  a mask entry of ln 2 == that key counted twice; -inf entries == deleting
  those keys; key order irrelevant; head h reads KV head h // (Nh / Nkv);
  q conversion to K's vec_dot type (fp16 / bf16 / Q8_0) idempotent and
  absent for F32 K, and for Q8_0 K it is the x86 quantizer (tie blocks);
  masked keys are never read (NaN there stays out); fully masked rows -> NaN;
  scores near 1000 stay finite. Planting each of these mistakes in a copy of
  the oracle fails at least one test: GQA map h % Nkv, no q conversion, the
  REF quantizer, no -inf skip, mask added before the scale, no max shift,
  the mask row of query 0 for every query, bf16 conversion done as fp16, 0
  instead of NaN for a fully masked row.
"""
import numpy as np
import pytest
from oracle import oracle as orc

LN2 = float(np.log(np.float32(2.0)))


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _fa(q, k, v, mask=None, scale=0.125, k_type="f32"):
    return orc.flash_attn_ext(q, k, v, mask, scale, k_type)


def test_single_key_returns_v():
    q, k, v = _rand((1, 2, 3, 64), 1), _rand((1, 1, 1, 64), 2), _rand((1, 1, 1, 64), 3)
    y = _fa(q, k, v)
    for iq in range(3):
        for h in range(2):
            assert np.array_equal(y[0, iq, h], v[0, 0, 0])


@pytest.mark.parametrize("how", ["q_zero", "scale_zero"])
def test_equal_scores_give_the_mean(how):
    q = np.zeros((1, 1, 2, 128), np.float32) if how == "q_zero" else _rand((1, 1, 2, 128), 4)
    k, v = _rand((1, 1, 37, 128), 5), _rand((1, 1, 37, 128), 6)
    y = _fa(q, k, v, scale=0.0 if how == "scale_zero" else 0.1)
    ref = v[0, 0].astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(y[0, 0, 0], ref, rtol=1e-6, atol=1e-7)


def test_mask_ln2_counts_a_key_twice():
    q, k, v = _rand((1, 1, 1, 64), 7), _rand((1, 1, 9, 64), 8), _rand((1, 1, 9, 64), 9)
    mask = np.zeros((1, 1, 1, 9), np.float32)
    mask[..., 4] = LN2
    y = _fa(q, k, v, mask)
    k2 = np.concatenate([k, k[:, :, 4:5]], axis=2)
    v2 = np.concatenate([v, v[:, :, 4:5]], axis=2)
    y2 = _fa(q, k2, v2)
    np.testing.assert_allclose(y, y2, rtol=2e-6, atol=1e-7)


def test_minus_inf_deletes_keys():
    q, k, v = _rand((2, 2, 3, 64), 10), _rand((2, 2, 20, 64), 11), _rand((2, 2, 20, 64), 12)
    drop = np.array([0, 3, 4, 19])
    mask = np.zeros((1, 1, 3, 20), np.float32)
    mask[..., drop] = -np.inf
    y = _fa(q, k, v, mask)
    keep = np.setdiff1d(np.arange(20), drop)
    y2 = _fa(q, k[:, :, keep], v[:, :, keep])
    np.testing.assert_allclose(y, y2, rtol=1e-6, atol=1e-7)


def test_key_order_irrelevant():
    q, k, v = _rand((1, 2, 2, 128), 13), _rand((1, 1, 50, 128), 14), _rand((1, 1, 50, 128), 15)
    mask = _rand((1, 1, 2, 50), 16)
    perm = np.random.default_rng(17).permutation(50)
    y = _fa(q, k, v, mask)
    y2 = _fa(q, k[:, :, perm], v[:, :, perm], np.ascontiguousarray(mask[..., perm]))
    np.testing.assert_allclose(y, y2, rtol=1e-6, atol=1e-7)


def test_gqa_head_mapping():
    N, Nh, Nkv, n_q, n_kv, D = 2, 6, 2, 2, 11, 64
    q, k, v = _rand((N, Nh, n_q, D), 18), _rand((N, Nkv, n_kv, D), 19), _rand((N, Nkv, n_kv, D), 20)
    y = _fa(q, k, v)
    for b in range(N):
        for h in range(Nh):
            g = h // (Nh // Nkv)
            one = _fa(q[b:b + 1, h:h + 1], k[b:b + 1, g:g + 1], v[b:b + 1, g:g + 1])
            assert np.array_equal(y[b, :, h], one[0, :, 0])


def test_mask_broadcast_over_heads_and_batch():
    N, Nh, n_q, n_kv = 4, 2, 3, 16
    q, k, v = _rand((N, Nh, n_q, 64), 21), _rand((N, 1, n_kv, 64), 22), _rand((N, 1, n_kv, 64), 23)
    mask = _rand((2, 1, 4, n_kv), 24)  # mN = 2 (b % 2), mQ = 4 >= n_q (padded)
    y = _fa(q, k, v, mask)
    for b in range(N):
        one = _fa(q[b:b + 1], k[b:b + 1], v[b:b + 1], np.ascontiguousarray(mask[b % 2:b % 2 + 1]))
        assert np.array_equal(y[b], one[0])


@pytest.mark.parametrize("k_type,conv", [("f16", lambda x: orc.f16_to_f32(orc.f32_to_f16(x))),
                                         ("bf16", lambda x: orc.bf16_to_f32(orc.f32_to_bf16(x))),
                                         ("q8_0", lambda x: orc.dequantize_q8_0(orc.quantize_q8_0(x, "x86")))])
def test_q_conversion(k_type, conv):
    q, k, v = _rand((1, 1, 2, 128), 25), _rand((1, 1, 30, 128), 26), _rand((1, 1, 30, 128), 27)
    y = _fa(q, k, v, k_type=k_type, scale=0.5)
    qc = conv(q)
    assert not np.array_equal(qc, q)
    assert np.array_equal(y, _fa(qc, k, v, k_type="f32", scale=0.5))  # the conversion is applied
    assert np.array_equal(y, _fa(qc, k, v, k_type=k_type, scale=0.5))  # and idempotent
    assert not np.array_equal(y, _fa(q, k, v, k_type="f32", scale=0.5))  # F32 K converts nothing


def test_fully_masked_row_is_nan():
    q, k, v = _rand((1, 1, 2, 64), 28), _rand((1, 1, 5, 64), 29), _rand((1, 1, 5, 64), 30)
    mask = np.zeros((1, 1, 2, 5), np.float32)
    mask[0, 0, 1] = -np.inf
    y = _fa(q, k, v, mask)
    assert np.isfinite(y[0, 0]).all() and np.isnan(y[0, 1]).all()


def test_large_scores_stay_finite():
    q, k, v = _rand((1, 1, 1, 64), 31, 40.0), _rand((1, 1, 64, 64), 32, 40.0), _rand((1, 1, 64, 64), 33)
    y = _fa(q, k, v, scale=1.0)  # scores of order 1e4: exp must be taken after the max shift
    assert np.isfinite(y).all()
    s = (q[0, 0, 0].astype(np.float64) @ k[0, 0].astype(np.float64).T)
    j = int(np.argmax(s))
    if np.sort(s)[-1] - np.sort(s)[-2] > 50:  # one key dominates by e^-50
        np.testing.assert_allclose(y[0, 0, 0], v[0, 0, j], rtol=1e-6, atol=1e-7)


def test_masked_keys_are_never_read():
    """ggml skips a -inf key before its dot product: NaN/inf in masked K or V rows
    must not reach the output."""
    q, k, v = _rand((1, 1, 2, 64), 34), _rand((1, 1, 12, 64), 35), _rand((1, 1, 12, 64), 36)
    mask = np.zeros((1, 1, 2, 12), np.float32)
    mask[..., [2, 7]] = -np.inf
    k[0, 0, 2] = np.nan
    v[0, 0, 7] = np.inf
    y = _fa(q, k, v, mask)
    assert np.isfinite(y).all()
    keep = np.setdiff1d(np.arange(12), [2, 7])
    np.testing.assert_allclose(y, _fa(q, k[:, :, keep], v[:, :, keep]), rtol=1e-6, atol=1e-7)


def test_q8_0_conversion_is_the_x86_quantizer():
    """Blocks with exact .5 ties after scaling (amax 127: id = 1) separate the
    x86 from_float (round half to even) from quantize_row_q8_0_ref (half away)."""
    blk = np.zeros(32, np.float32)
    blk[0] = 127.0
    blk[1:] = (np.arange(1, 32) % 9).astype(np.float32) + 0.5
    q = np.tile(blk, 4).reshape(1, 1, 1, 128)
    k, v = _rand((1, 1, 20, 128), 37), _rand((1, 1, 20, 128), 38)
    x86 = orc.dequantize_q8_0(orc.quantize_q8_0(q, "x86"))
    ref = orc.dequantize_q8_0(orc.quantize_q8_0(q, "ref"))
    assert not np.array_equal(x86, ref)
    y = _fa(q, k, v, k_type="q8_0", scale=0.01)
    assert np.array_equal(y, _fa(x86, k, v, k_type="f32", scale=0.01))
    assert not np.array_equal(y, _fa(ref, k, v, k_type="f32", scale=0.01))


# ---------------------------------------------------------------------------
# ggml-cpu's F16-V variant (orc_flash_attn_ext_f16acc): the output accumulated
# in fp16 one key at a time
# ---------------------------------------------------------------------------
def _f16(x):
    return orc.f32_to_f16(np.asarray(x, np.float32))


def test_f16acc_exact_when_every_partial_sum_is_an_fp16_integer():
    """q = 0: every score is 0, vs = 1, S = n; small integer V keeps every
    partial sum an integer below 2048, so nothing rounds: y = sum(v) * (1/n)
    and the budget is 0."""
    r = np.random.default_rng(3)
    n, D = 300, 64
    v = r.integers(-3, 4, (1, 1, n, D)).astype(np.float32)
    k = _rand((1, 1, n, D), 4)
    q = np.zeros((1, 2, 1, D), np.float32)
    y, bud = orc.flash_attn_ext_f16acc(q, k, _f16(v), None, 0.125)
    want = v[0, 0].sum(axis=0).astype(np.float32) * np.float32(1.0 / np.float32(n))
    for h in range(2):
        assert np.array_equal(y[0, 0, h], want)
    assert not bud.any()


def test_f16acc_stalls_at_2048_like_fp16():
    """V = 1 for 3000 keys of equal score: the fp16 count reaches 2048, where
    2048 + 1 rounds back to 2048 (ties to even), so y = 2048 * (1/3000) while
    the exact value is 1. An fp32 accumulation would give 1."""
    n, D = 3000, 32
    q = np.zeros((1, 1, 1, D), np.float32)
    k = _rand((1, 1, n, D), 5)
    v = np.ones((1, 1, n, D), np.float32)
    y, bud = orc.flash_attn_ext_f16acc(q, k, _f16(v), None, 0.125)
    assert np.all(y == np.float32(2048.0) * np.float32(np.float32(1.0) / np.float32(n)))
    assert np.allclose(bud, (n - 2048) / n, rtol=1e-6)
    assert np.all(orc.flash_attn_ext(q, k, v, None, 0.125) == 1.0)


@pytest.mark.parametrize("n_kv", [40, 700, 4096])
def test_f16acc_within_its_budget_of_the_exact_value(n_kv):
    """Random scores, masks and V: the fp16 result differs from the exact
    value by at most its own carried rounding errors plus the fp32 softmax's
    (1e-5 of the output scale); and masked keys drop out as in the exact oracle."""
    N, Nh, Nkv, n_q, D = 2, 4, 2, 3, 128
    q, k = _rand((N, Nh, n_q, D), 6), _rand((N, Nkv, n_kv, D), 7)
    v16 = _f16(_rand((N, Nkv, n_kv, D), 8))
    vf = orc.f16_to_f32(v16)
    m = np.where(np.random.default_rng(9).random((N, 1, n_q, n_kv)) < 0.3, -np.inf, 0.0).astype(np.float32)
    m[..., 0] = 0.0
    y, bud = orc.flash_attn_ext_f16acc(q, k, v16, m, 1.0 / np.sqrt(D))
    ref = orc.flash_attn_ext(q, k, vf, m, 1.0 / np.sqrt(D), "f16")
    assert np.all(np.abs(y - ref) <= bud + 1e-5 * np.abs(vf).max())
    assert bud.max() > 0
