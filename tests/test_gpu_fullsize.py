"""GPU parity at the benchmark configurations' full sizes.

The oracle is fast enough on the host to run the full shapes, so these
compare every element, at the same bars as the small-shape tests:
  C3  ACE-Step DiT block, bf16, 12000 rows x 2048 (the 5 fused launches the
      benchmark times): <= 1 bf16 ulp (row floor for rope and modulate, whose
      outputs can cancel), residual sums bit-exact
  C4  Qwen3-1.7B prefill: Q8_0 embedding get_rows from a 151669 x 2048 table
      for 16384 ids (bit-exact) and the FP16-range residual add+clamp with
      outliers (bit-exact)
  C5  Qwen3-4B prefill into a Q8_0 KV cache: K, V [8, 2048, 8, 128] quantized
      at slot offsets U[0, 6144) of an 8192-slot cache (int8 quants and fp16
      scales bit-exact), then dequantized back through get_rows (bit-exact)
  C4, C5 F32 QK-norm -> rope over all 16384 tokens (16/8 and 32/8 heads): the
      persistent kernel's multi-item walk, <= 1e-5 with the row floor; C5 as
      the chain the configuration describes: QK-norm + rope from the fused QKV
      output, the kernel's own K and the V view stored as Q8_0 (bit-exact
      against the oracle quantizing those very values), then gathered back
"""
import os

import numpy as np
import pytest

from helpers import assert_bf16_ulp, assert_f32_close, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import Q8_0_CPU_X86, ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu
EPS = 1e-6


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    orc.set_threads(max(1, min(os.cpu_count() or 1, 16)))
    yield
    orc.set_threads(1)


def _normal(rng, shape, scale=1.0, mean=0.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale) + np.float32(mean)).astype(np.float32)


def test_c3_dit_block_full_size(dev):
    print("full size C3: DiT block bf16, 12000 x 2048", flush=True)
    R, H, NH, NKV, D, I, T = 12000, 2048, 16, 8, 128, 6144, 6000
    rng = np.random.default_rng(42)
    hid = orc.f32_to_bf16(_normal(rng, (R, H)))
    qkv = orc.f32_to_bf16(_normal(rng, (R, (NH + 2 * NKV) * D)))
    sa_out = orc.f32_to_bf16(_normal(rng, (R, H)))
    gate_up = orc.f32_to_bf16(_normal(rng, (R, 2 * I)))
    ffn_out = orc.f32_to_bf16(_normal(rng, (R, H)))
    ad = _normal(rng, (6 * H,), 0.1)
    sa_w, ff_w = _normal(rng, (H,), 0.1, 1.0), _normal(rng, (H,), 0.1, 1.0)
    q_w, k_w = _normal(rng, (D,), 0.1, 1.0), _normal(rng, (D,), 0.1, 1.0)
    pos = np.tile(np.arange(T, dtype=np.int32), R // T)
    shift_sa, scale_sa, gate_sa, shift_ff, scale_ff, gate_ff = (ad[i * H:(i + 1) * H] for i in range(6))

    d_h, d_qkv, d_sa, d_gu, d_ffo = (to_dev(a, bf16=True) for a in (hid, qkv, sa_out, gate_up, ffn_out))
    d_ad, d_saw, d_ffw, d_qw, d_kw, d_pos = (to_dev(a) for a in (ad, sa_w, ff_w, q_w, k_w, pos))
    vec = lambda i: d_ad[i * H:(i + 1) * H]  # noqa: E731
    q = d_qkv[:, :NH * D].unflatten(1, (NH, D))
    k = d_qkv[:, NH * D:(NH + NKV) * D].unflatten(1, (NKV, D))
    norm_sa = ops.rms_norm_modulate(d_h, d_saw, vec(1), vec(0), EPS)
    q_out, k_out = ops.qk_norm_rope(q, d_qw, d_pos, EPS, D, 1e4, k=k, k_w=d_kw)
    h1, norm_ff = ops.add_rms_norm(d_h, d_sa, EPS, gate=vec(2), w=d_ffw, scale=vec(4), shift=vec(3))
    ff = ops.swiglu(d_gu)
    h2 = ops.gated_add(h1, d_ffo, vec(5))

    ch = orc.bf16_chain
    assert_bf16_ulp(to_np(norm_sa), ch(orc.rms_norm_modulate, hid, sa_w, scale_sa, shift_sa, EPS), row_floor=True)
    qh = qkv[:, :NH * D].reshape(R, NH, D)
    kh = qkv[:, NH * D:(NH + NKV) * D].reshape(R, NKV, D)
    assert_bf16_ulp(to_np(q_out), ch(orc.qk_norm_rope, qh, q_w, pos, EPS, D, 1e4), row_floor=True)
    assert_bf16_ulp(to_np(k_out), ch(orc.qk_norm_rope, kh, k_w, pos, EPS, D, 1e4), row_floor=True)
    h1_ref = ch(orc.gated_add, hid, sa_out, gate_sa)
    assert np.array_equal(to_np(h1), h1_ref)
    assert_bf16_ulp(to_np(norm_ff), ch(orc.rms_norm_modulate, h1_ref, ff_w, scale_ff, shift_ff, EPS),
                    row_floor=True)
    assert_bf16_ulp(to_np(ff), ch(orc.swiglu, gate_up))
    assert np.array_equal(to_np(h2), ch(orc.gated_add, h1_ref, ffn_out, gate_ff))


def test_c4_embedding_and_clamp_full_size(dev):
    print("full size C4: Q8_0 get_rows 151669 x 2048, 16384 ids; add+clamp 16384 x 2048", flush=True)
    n_rows, H, T = 151669, 2048, 16384
    rng = np.random.default_rng(4)
    rb = H // 32 * 34
    table = np.empty((n_rows, rb), np.uint8)
    for r0 in range(0, n_rows, 16384):  # built in chunks: only the Q8_0 bytes are kept
        r1 = min(n_rows, r0 + 16384)
        table[r0:r1] = orc.quantize_q8_0(_normal(rng, (r1 - r0, H), 0.02), "ref")
    ids = rng.integers(0, n_rows, T).astype(np.int32)
    ids[:2] = [0, n_rows - 1]
    y = to_np(ops.get_rows(ops.Q8(to_dev(table)), to_dev(ids)))
    assert np.array_equal(y.view(np.uint32), orc.get_rows(table, orc.Q8_0, H, ids).view(np.uint32))
    del table

    a, b = _normal(rng, (T, H)), _normal(rng, (T, H))
    idx = rng.choice(a.size, a.size // 1000, replace=False)
    a.reshape(-1)[idx] = _normal(rng, (idx.size,), 1000.0)
    a.reshape(-1)[rng.choice(a.size, 16, replace=False)] = np.float32(1e5)
    y = to_np(ops.add_clamp(to_dev(a), to_dev(b)))
    assert np.array_equal(y.view(np.uint32), orc.add_clamp(a, b).view(np.uint32))


def test_c5_kv_store_q8_0_full_size(dev):
    print("full size C5: K,V [8,2048,8,128] f32 -> Q8_0 cache 8192 slots, then get_rows back", flush=True)
    B, T, NKV, D, max_seq = 8, 2048, 8, 128, 8192
    rng = np.random.default_rng(5)
    k, v = _normal(rng, (B, T, NKV, D)), _normal(rng, (B, T, NKV, D))
    s0 = rng.integers(0, 6144, B).astype(np.int32)
    rb = D // 32 * 34
    kc = DTensor.full_byte((B, NKV, max_seq, rb), 0xA5)
    vc = DTensor.full_byte((B, NKV, max_seq, rb), 0x5A)
    ops.kv_store(to_dev(k), ops.Q8(kc), to_dev(s0), v=to_dev(v), v_cache=ops.Q8(vc), rounding=Q8_0_CPU_X86)
    kch, vch = to_np(kc), to_np(vc)
    written = np.zeros((B, NKV, max_seq), bool)
    for b in range(B):
        written[b, :, s0[b]:s0[b] + T] = True
        for src, cache in ((k, kch), (v, vch)):
            want = orc.quantize_q8_0(np.ascontiguousarray(src[b].transpose(1, 0, 2)), "x86")  # (NKV, T, rb)
            assert np.array_equal(cache[b, :, s0[b]:s0[b] + T], want), f"sequence {b}"
    assert (kch[~written] == 0xA5).all() and (vch[~written] == 0x5A).all()
    ids = np.flatnonzero(written.reshape(-1)).astype(np.int32)
    for cache_d, cache_h in ((kc, kch), (vc, vch)):
        y = to_np(ops.get_rows(ops.Q8(cache_d.view(-1, rb)), to_dev(ids)))
        assert np.array_equal(y.view(np.uint32), orc.dequantize_q8_0(cache_h.reshape(-1, rb)[ids]).view(np.uint32))


def _qkv_rope(rng, B, T, NH, NKV, D, theta, pos):
    R = B * T
    qkv = _normal(rng, (R, (NH + 2 * NKV) * D))
    q_w, k_w = _normal(rng, (D,), 0.1, 1.0), _normal(rng, (D,), 0.1, 1.0)
    d_qkv = to_dev(qkv)
    q = d_qkv[:, :NH * D].unflatten(1, (NH, D))
    k = d_qkv[:, NH * D:(NH + NKV) * D].unflatten(1, (NKV, D))
    q_out, k_out = ops.qk_norm_rope(q, to_dev(q_w), to_dev(pos), EPS, D, theta, k=k, k_w=to_dev(k_w))
    return qkv, q_w, k_w, d_qkv, q_out, k_out


def _check_rope(qkv, q_w, k_w, q_out, k_out, NH, NKV, D, theta, pos):
    R = qkv.shape[0]
    qh = qkv[:, :NH * D].reshape(R, NH, D)
    kh = qkv[:, NH * D:(NH + NKV) * D].reshape(R, NKV, D)
    ko = to_np(k_out)
    assert_f32_close(to_np(q_out), orc.qk_norm_rope(qh, q_w, pos, EPS, D, theta), row_floor=True)
    assert_f32_close(ko, orc.qk_norm_rope(kh, k_w, pos, EPS, D, theta), row_floor=True)
    return ko


def test_c4_qk_norm_rope_f32_full_size(dev):
    print("full size C4: F32 QK-norm -> rope, 4 x 4096 tokens, 16/8 heads x 128", flush=True)
    B, T, NH, NKV, D = 4, 4096, 16, 8, 128
    rng = np.random.default_rng(44)
    pos = np.tile(np.arange(T, dtype=np.int32), B)
    qkv, q_w, k_w, _, q_out, k_out = _qkv_rope(rng, B, T, NH, NKV, D, 1e6, pos)
    _check_rope(qkv, q_w, k_w, q_out, k_out, NH, NKV, D, 1e6, pos)


def test_c5_rope_store_gather_chain_full_size(dev):
    print("full size C5 chain: F32 QK-norm -> rope (8 x 2048, 32/8 heads), K/V -> Q8_0 cache, get_rows back",
          flush=True)
    B, T, NH, NKV, D, max_seq = 8, 2048, 32, 8, 128, 8192
    rng = np.random.default_rng(55)
    s0 = rng.integers(0, 6144, B).astype(np.int32)
    pos = (s0[:, None] + np.arange(T, dtype=np.int32)[None, :]).reshape(-1)  # kv_pos + i (qwen3-lm.h:516-522)
    qkv, q_w, k_w, d_qkv, q_out, k_out = _qkv_rope(rng, B, T, NH, NKV, D, 1e6, pos)
    ko = _check_rope(qkv, q_w, k_w, q_out, k_out, NH, NKV, D, 1e6, pos)
    v_dev = d_qkv[:, (NH + NKV) * D:].unflatten(1, (NKV, D)).unflatten(0, (B, T))
    rb = D // 32 * 34
    kc = DTensor.full_byte((B, NKV, max_seq, rb), 0xA5)
    vc = DTensor.full_byte((B, NKV, max_seq, rb), 0x5A)
    ops.kv_store(k_out.unflatten(0, (B, T)), ops.Q8(kc), to_dev(s0), v=v_dev, v_cache=ops.Q8(vc),
                 rounding=Q8_0_CPU_X86)
    kch, vch = to_np(kc), to_np(vc)
    k_src = ko.reshape(B, T, NKV, D)
    v_src = qkv[:, (NH + NKV) * D:].reshape(B, T, NKV, D)
    for b in range(B):
        for src, cache in ((k_src, kch), (v_src, vch)):
            want = orc.quantize_q8_0(np.ascontiguousarray(src[b].transpose(1, 0, 2)), "x86")
            assert np.array_equal(cache[b, :, s0[b]:s0[b] + T], want), f"sequence {b}"
    ids = np.concatenate([((b * NKV + h) * max_seq + s0[b] + np.arange(T)) for b in range(B) for h in range(NKV)])
    ids = ids.astype(np.int32)
    for cache_d, src in ((kc, k_src), (vc, v_src)):
        y = to_np(ops.get_rows(ops.Q8(cache_d.view(-1, rb)), to_dev(ids)))
        want = orc.dequantize_q8_0(orc.quantize_q8_0(np.ascontiguousarray(src.transpose(0, 2, 1, 3)), "x86"))
        assert np.array_equal(y.view(np.uint32), want.reshape(-1, D).view(np.uint32))
