"""GPU: mi_qk_norm_rope_kv_store (QK-norm -> rope and the KV-cache store in one
launch) against the three calls it replaces, mi_qk_norm_rope -> [mi_add_clamp
on V] -> mi_kv_store, on the same inputs. Bar, written here: bit-identical --
q_out, every byte of both caches (untouched slots keep their sentinel bytes)
and the bad-slot count. The separate calls are themselves checked against the
oracle (test_gpu_rope.py, test_gpu_q8.py, test_gpu_qwen3_layer.py); one case
here also checks the fused result against the oracle chain directly.
"""
import numpy as np
import pytest
from helpers import bf16_ordinal, randn, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import _lib, ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu

Q8 = "q8_0"


def _cache(shape_rows, ctype, fill):
    """cache of (n_sets, Nkv, max_seq, D) in ctype, every byte = fill"""
    n_sets, nkv, max_seq, D = shape_rows
    if ctype == Q8:
        return ops.Q8(DTensor.full_byte((n_sets, nkv, max_seq, D // 32 * 34), fill))
    return DTensor.full_byte((n_sets, nkv, max_seq, D), fill, ctype)


def _bytes(c):
    return np.ascontiguousarray(to_np(c.data if isinstance(c, ops.Q8) else c)).view(np.uint8)


def _run(dt, ctype, D, B, T, nh, nkv, *, clamp=False, rounding=_lib.Q8_0_CPU_X86, bad=False, seed=0, fused_qkv=True,
         theta=1e6):
    r = np.random.default_rng(seed)
    n_tok = B * T
    width = (nh + 2 * nkv) * D
    x = randn((n_tok, width), seed=seed + 1)
    if clamp:  # V outliers beyond the fp16 range
        idx = r.integers(0, n_tok * nkv * D, 40)
        x[idx // (nkv * D), (nh + nkv) * D + idx % (nkv * D)] = r.choice([-1.5e5, 1.5e5, 7e4, -7e4], 40)
    xd = to_dev(orc.f32_to_bf16(x), bf16=True) if dt == "bf16" else to_dev(x)
    if fused_qkv:
        q = xd[:, :nh * D].unflatten(1, (nh, D))
        k = xd[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
        v = xd[:, (nh + nkv) * D:].unflatten(1, (nkv, D))
    else:
        q = to_dev(np.ascontiguousarray(to_np(xd)[:, :nh * D])).view(n_tok, nh, D) if dt == "f32" else \
            to_dev(np.ascontiguousarray(to_np(xd)[:, :nh * D]), bf16=True).view(n_tok, nh, D)
        k = xd[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
        v = xd[:, (nh + nkv) * D:].unflatten(1, (nkv, D))
    qw = to_dev(randn(D, seed=seed + 2, scale=0.1, mean=1.0))
    kw = to_dev(randn(D, seed=seed + 3, scale=0.1, mean=1.0))
    pos = to_dev(r.integers(0, 8192, n_tok).astype(np.int32))
    max_seq, n_sets = 256, B + 1
    p0 = r.integers(0, max_seq - T + 1, B).astype(np.int32)
    sets = r.permutation(n_sets)[:B].astype(np.int32)
    if bad:
        p0[0] = max_seq - T + 1  # the last token of sequence 0 is out of range
        sets[-1] = n_sets + 3    # every token of the last sequence is out of range
    pos0, setd = to_dev(p0), to_dev(sets)
    shape = (n_sets, nkv, max_seq, D)

    # the three calls
    kc0, vc0 = _cache(shape, ctype, 0xA5), _cache(shape, ctype, 0x5A)
    e0 = DTensor.zeros((1,), "i32")
    q_ref, k_ref = ops.qk_norm_rope(q, qw, pos, 1e-6, D, theta, k=k, k_w=kw)
    v_src = v
    if clamp:
        v_src = ops.add_clamp(v, None, -65504.0, 65504.0)
    ops.kv_store(k_ref.unflatten(0, (B, T)), kc0, pos0, v=v_src.unflatten(0, (B, T)), v_cache=vc0, sets=setd,
                 rounding=rounding, err=e0)
    # the fused call
    kc1, vc1 = _cache(shape, ctype, 0xA5), _cache(shape, ctype, 0x5A)
    e1 = DTensor.zeros((1,), "i32")
    v_before = to_np(v)
    q_f = ops.qk_norm_rope_kv_store(q, qw, k, kw, v, pos, 1e-6, D, theta, kc1, vc1, pos0, sets=setd, clamp_v=clamp,
                                    rounding=rounding, err=e1)
    assert np.array_equal(to_np(q_f), to_np(q_ref)), "q_out"
    assert np.array_equal(_bytes(kc1), _bytes(kc0)), "k cache"
    assert np.array_equal(_bytes(vc1), _bytes(vc0)), "v cache"
    assert int(to_np(e1)[0]) == int(to_np(e0)[0])
    assert np.array_equal(to_np(v), v_before), "v is not modified"
    if bad:
        assert int(to_np(e1)[0]) == 2 * nkv * (1 + T)
    return x, p0, sets, q_f, kc1, to_np(pos)


@pytest.mark.parametrize("rounding", [_lib.Q8_0_CPU_X86, _lib.Q8_0_REF])
@pytest.mark.parametrize("clamp", [False, True])
def test_qwen3_4b_decode_q8_cache(dev, rounding, clamp):
    """Qwen3-4B decode: batch 8, one token each, 32/8 heads x 128, bf16, Q8_0 cache"""
    print(f"qk rope kv fused C2 rounding={rounding} clamp={clamp}", flush=True)
    _run("bf16", Q8, 128, 8, 1, 32, 8, clamp=clamp, rounding=rounding, seed=rounding * 2 + clamp)


@pytest.mark.parametrize("dt,ctype", [("f32", "f16"), ("f32", Q8), ("bf16", "f16"), ("bf16", "bf16"),
                                      ("f32", "f32"), ("bf16", "f32")])
def test_prefill_chunks_and_cache_types(dev, dt, ctype):
    """3 sequences x 5 tokens, the reference's F16 cache and the others"""
    print(f"qk rope kv fused {dt} -> {ctype}", flush=True)
    _run(dt, ctype, 128, 3, 5, 16, 8, seed=7)


@pytest.mark.parametrize("D,nh,nkv", [(64, 8, 2), (256, 8, 4)])
def test_head_sizes(dev, D, nh, nkv):
    print(f"qk rope kv fused D={D}", flush=True)
    _run("bf16", Q8, D, 4, 2, nh, nkv, seed=D)
    _run("f32", "f16", D, 2, 3, nh, nkv, seed=D + 1, theta=1e4)


def test_bad_slots_and_contiguous_q(dev):
    print("qk rope kv fused bad slots", flush=True)
    _run("bf16", Q8, 128, 4, 3, 16, 8, bad=True, seed=9, fused_qkv=False)
    _run("f32", "f16", 128, 4, 3, 16, 8, bad=True, seed=10)


def test_against_oracle_chain(dev):
    """the fused result against the oracle directly: Q within 1 bf16 ulp of the
    oracle's QK-norm -> rope, and the V cache rows bit-exact against the oracle's
    x86 Q8_0 quantizer on the bf16 V rows (K goes through the rope, whose bf16
    output may differ by an ulp; the three-call comparison above pins it)"""
    print("qk rope kv fused vs oracle", flush=True)
    B, T, nh, nkv, D = 8, 1, 32, 8, 128
    x, p0, sets, q_f, kc, pos = _run("bf16", Q8, D, B, T, nh, nkv, seed=21)
    xb = orc.bf16_to_f32(orc.f32_to_bf16(x))
    qh = xb[:, :nh * D].reshape(B * T, nh, D)
    qw = randn(D, seed=21 + 2, scale=0.1, mean=1.0)
    want = orc.f32_to_bf16(orc.qk_norm_rope(qh, qw, pos, 1e-6, D, 1e6))
    d = np.abs(bf16_ordinal(to_np(q_f)).astype(np.int64) - bf16_ordinal(want).astype(np.int64))
    assert d.max() <= 1


def test_v_cache_against_oracle(dev):
    print("qk rope kv fused V vs oracle", flush=True)
    r = np.random.default_rng(5)
    B, T, nh, nkv, D = 8, 1, 32, 8, 128
    x = randn((B * T, (nh + 2 * nkv) * D), seed=31)
    xd = to_dev(orc.f32_to_bf16(x), bf16=True)
    q = xd[:, :nh * D].unflatten(1, (nh, D))
    k = xd[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
    v = xd[:, (nh + nkv) * D:].unflatten(1, (nkv, D))
    w = to_dev(np.ones(D, np.float32))
    pos = to_dev(r.integers(0, 8192, B * T).astype(np.int32))
    p0 = r.integers(0, 100, B).astype(np.int32)
    kc, vc = _cache((B, nkv, 128, D), Q8, 0), _cache((B, nkv, 128, D), Q8, 0)
    ops.qk_norm_rope_kv_store(q, w, k, w, v, pos, 1e-6, D, 1e6, kc, vc, to_dev(p0))
    vch = _bytes(vc).reshape(B, nkv, 128, D // 32 * 34)
    vb = orc.bf16_to_f32(orc.f32_to_bf16(x))[:, (nh + nkv) * D:].reshape(B, nkv, D)
    for b in range(B):
        assert np.array_equal(vch[b, :, p0[b]], orc.quantize_q8_0(vb[b], "x86")), f"b={b}"
