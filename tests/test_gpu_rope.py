"""GPU parity: per-head QK-RMSNorm -> NEOX rope (and plain rope) vs the oracle.

Rotated outputs are differences that can cancel, so the fp32 bar is
|a - ref| <= 1e-5 * max(|ref|, rms(ref head row)); cos/sin come from the
device libm (ocml) vs glibc and may differ in the last ulp.
bf16: within 1 ulp of the oracle's RNE-rounded result.
"""
import numpy as np
import pytest
from helpers import assert_bf16_ulp, assert_f32_close, frac_bitexact, randn, rng, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _fused_qkv(T, nh, nkv, D, seed, bf16, dev):
    """Q/K/V as strided views of one [T, (nh + 2 nkv) * D] projection output."""
    qkv = randn((T, (nh + 2 * nkv) * D), seed=seed)
    host = orc.f32_to_bf16(qkv) if bf16 else qkv
    d = to_dev(host, dev, bf16=bf16)
    q = d[:, : nh * D].unflatten(1, (nh, D))
    k = d[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
    qh = host[:, : nh * D].reshape(T, nh, D)
    kh = host[:, nh * D:(nh + nkv) * D].reshape(T, nkv, D)
    return q, k, qh, kh


def _check(out, ref_f32_fn, host_in, bf16):
    if bf16:
        assert_bf16_ulp(to_np(out), orc.bf16_chain(ref_f32_fn, host_in), row_floor=True)
    else:
        assert_f32_close(to_np(out), ref_f32_fn(host_in), row_floor=True)


@pytest.mark.parametrize("T,nh,nkv,D,theta,maxpos", [
    (512, 16, 8, 128, 1e6, 512),      # Qwen3-0.6B prefill
    (8, 32, 8, 128, 1e6, 8192),       # Qwen3-4B decode, positions ~U[0, 8191]
    (300, 16, 8, 128, 1e4, 300),      # DiT self-attn (frame index)
    (64, 4, 2, 64, 1e4, 4096),
    (50, 2, 1, 256, 1e6, 40000),
])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_qk_norm_rope_fused_qkv(dev, T, nh, nkv, D, theta, maxpos, dt):
    print(f"qk_norm_rope T={T} nh={nh} nkv={nkv} D={D} theta={theta} {dt}", flush=True)
    bf16 = dt == "bf16"
    q, k, qh, kh = _fused_qkv(T, nh, nkv, D, seed=T + D, bf16=bf16, dev=dev)
    pos = rng(5).integers(0, maxpos, T).astype(np.int32)
    if maxpos == T:
        pos = np.arange(T, dtype=np.int32)
    qw = randn((D,), seed=1, scale=0.1, mean=1.0)
    kw = randn((D,), seed=2, scale=0.1, mean=1.0)
    qo, ko = ops.qk_norm_rope(q, to_dev(qw, dev), to_dev(pos, dev), EPS, D, theta, k=k, k_w=to_dev(kw, dev))
    _check(qo, lambda a: orc.qk_norm_rope(a, qw, pos, EPS, D, theta), qh, bf16)
    _check(ko, lambda a: orc.qk_norm_rope(a, kw, pos, EPS, D, theta), kh, bf16)


@pytest.mark.parametrize("nh,nkv,dt", [
    (16, 16, "bf16"),  # 4 batches of 8 rows, 2 per work item
    (16, 8, "bf16"),   # DiT self-attention (16 Q, 8 KV heads): 3 batches, a whole token per item
    (24, 16, "bf16"),  # 5 batches, items of 3 + 2
    (14, 6, "bf16"),   # heads not a multiple of the batch: rows past the last head
    (6, 2, "f32"),     # f32 rows (batches of 4): 2 + 1 batches, ragged Q rows
])
def test_qk_norm_rope_long_sequences_group_batches(dev, nh, nkv, dt):
    """2100 tokens: enough to fill the chip with whole tokens, so each wave item
    holds several head batches (2 or 3), including ragged last items and rows."""
    T, D, theta = 2100, 128, 1e4
    print(f"qk_norm_rope long T={T} nh={nh} nkv={nkv} {dt}", flush=True)
    bf16 = dt == "bf16"
    q, k, qh, kh = _fused_qkv(T, nh, nkv, D, seed=nh * 100 + nkv, bf16=bf16, dev=dev)
    pos = np.arange(T, dtype=np.int32)[::-1].copy()
    qw = randn((D,), seed=3, scale=0.1, mean=1.0)
    kw = randn((D,), seed=4, scale=0.1, mean=1.0)
    qo, ko = ops.qk_norm_rope(q, to_dev(qw, dev), to_dev(pos, dev), EPS, D, theta, k=k, k_w=to_dev(kw, dev))
    _check(qo, lambda a: orc.qk_norm_rope(a, qw, pos, EPS, D, theta), qh, bf16)
    _check(ko, lambda a: orc.qk_norm_rope(a, kw, pos, EPS, D, theta), kh, bf16)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_rope_only_and_4d_batch(dev, dt):
    """ggml_rope_ext on [D, H, S, N] (positions index S, reused for each N)."""
    bf16 = dt == "bf16"
    N, S, H, D = 2, 40, 3, 128
    x = randn((N, S, H, D), seed=9)
    host = orc.f32_to_bf16(x) if bf16 else x
    pos = np.arange(S, dtype=np.int32) * 3
    y = ops.rope_ext(to_dev(host, dev, bf16=bf16), to_dev(pos, dev), D, 2, 1e4)
    _check(y, lambda a: orc.rope_neox(a, pos, D, 1e4), host, bf16)


def test_qk_norm_bf16_generic_path_matches_fast_path(dev):
    """QK-norm -> rope on a BF16 view 2 bytes off 16-byte alignment (the generic
    kernel) and on its aligned copy (the fast one): both sum each head row's
    squares in fp32, in different orders, so each is within 1 ulp of the oracle
    and of the other, and almost all outputs are bit-identical."""
    T, nh, D = 40, 16, 128
    xb = orc.f32_to_bf16(randn((T * nh * D + 1,), seed=31))
    w = randn((D,), seed=32, scale=0.1, mean=1.0)
    pos = rng(33).integers(0, 4096, T).astype(np.int32)
    wd, pd = to_dev(w, dev), to_dev(pos, dev)
    un = to_dev(xb, dev, bf16=True)[1:].view(T, nh, D)
    al = to_dev(np.ascontiguousarray(xb[1:]).reshape(T, nh, D), dev, bf16=True)
    yg = to_np(ops.qk_norm_rope(un, wd, pd, EPS, D, 1e6)[0])
    yf = to_np(ops.qk_norm_rope(al, wd, pd, EPS, D, 1e6)[0])
    ref = orc.bf16_chain(lambda a: orc.qk_norm_rope(a, w, pos, EPS, D, 1e6), xb[1:].reshape(T, nh, D))
    assert_bf16_ulp(yg, ref, row_floor=True)
    assert_bf16_ulp(yf, ref, row_floor=True)
    assert_bf16_ulp(yg, yf, row_floor=True)
    assert frac_bitexact(yg, yf) >= 0.99


def test_rope_partial_dims_generic(dev):
    """n_dims < ne0 (remaining dims copied) and a non-{64,128,256} head size."""
    x = randn((20, 4, 128), seed=1)
    pos = rng(2).integers(0, 5000, 20).astype(np.int32)
    y = ops.rope_ext(to_dev(x, dev), to_dev(pos, dev), 64, 2, 1e6)
    assert_f32_close(to_np(y), orc.rope_neox(x, pos, 64, 1e6), row_floor=True)
    x = randn((20, 4, 96), seed=3)
    y = ops.rope_ext(to_dev(x, dev), to_dev(pos, dev), 96, 2, 1e6)
    assert_f32_close(to_np(y), orc.rope_neox(x, pos, 96, 1e6), row_floor=True)


def test_rope_scaling_params(dev):
    x = randn((16, 2, 128), seed=4)
    pos = np.arange(16, dtype=np.int32) * 100
    y = ops.rope_ext(to_dev(x, dev), to_dev(pos, dev), 128, 2, 1e6, freq_scale=0.25, attn_factor=1.5)
    assert_f32_close(to_np(y), orc.rope_neox(x, pos, 128, 1e6, 0.25, 1.5), row_floor=True)


def test_rope_position_zero_is_identity(dev):
    x = randn((4, 8, 128), seed=6)
    pos = np.zeros(4, np.int32)
    y = to_np(ops.rope_ext(to_dev(x, dev), to_dev(pos, dev), 128, 2, 1e6))
    assert np.array_equal(y, x)


@pytest.mark.parametrize("ne0,n_dims", [(128, 128), (96, 64)])
def test_rope_huge_positions_take_library_path(dev, ne0, n_dims):
    """Angles |x| >= 2^20 (positions past 2^20) use the math library's sincosf;
    positions below stay on the in-kernel reduction. Both against glibc."""
    x = randn((6, 4, ne0), seed=9)
    pos = np.array([3, 1048575, 1048576, 3000017, 123456789, 2147483000], np.int32)
    y = to_np(ops.qk_norm_rope(to_dev(x, dev), to_dev(randn((ne0,), seed=10, scale=0.1, mean=1.0), dev),
                               to_dev(pos, dev), EPS, n_dims, 1e6)[0])
    ref = orc.qk_norm_rope(x, randn((ne0,), seed=10, scale=0.1, mean=1.0), pos, EPS, n_dims, 1e6)
    assert_f32_close(y, ref, row_floor=True)


def test_qk_norm_no_rope_cross_attn(dev):
    """Cross-attention QK-norm: rms_norm(x) * w on [D, S, H, N] permuted views."""
    N, S, H, D = 2, 30, 8, 128
    x = to_dev(randn((N, S, H, D), seed=7), dev).permute(0, 2, 1, 3)  # (N, H, S, D): strided view
    w = randn((D,), seed=8, scale=0.1, mean=1.0)
    y = ops.rms_norm(x, EPS, w=to_dev(w, dev))
    assert_f32_close(to_np(y), orc.rms_norm_mul(to_np(x), w, EPS))


@pytest.mark.parametrize("H", [16, 20])
def test_qk_norm_no_rope_long_rows(dev, H):
    """Per-head Q-norm on 4400 x H x 128 bf16 (the cross-attention query shape):
    2 or 3 head batches per work item, and with 20 heads rows past the last
    head of a batch."""
    rows, D = 4400, 128
    print(f"q-norm long rows={rows} H={H}", flush=True)
    xb = orc.f32_to_bf16(randn((rows, H, D), seed=H))
    w = randn((D,), seed=11, scale=0.1, mean=1.0)
    y = ops.rms_norm(to_dev(xb, dev, bf16=True), EPS, w=to_dev(w, dev))
    assert_bf16_ulp(to_np(y), orc.bf16_chain(lambda a: orc.rms_norm_mul(a, w, EPS), xb), row_floor=True)


def test_rope_unsupported_modes_rejected(dev):
    x = to_dev(randn((4, 2, 128), seed=1), dev)
    pos = to_dev(np.arange(4, dtype=np.int32), dev)
    with pytest.raises(ops._lib.MiError):
        ops.rope_ext(x, pos, 128, 0, 1e4)  # NORMAL mode
    with pytest.raises(ops._lib.MiError):
        ops.rope_ext(x, pos, 128, 2, 1e4, ext_factor=1.0)
