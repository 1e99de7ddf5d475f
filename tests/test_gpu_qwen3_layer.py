"""A whole Qwen3 decode layer on the device (acestep_ops.qwen3.Qwen3DecodeLayer:
norm, Q8_0 QKV product, QK-norm + rope, KV-cache write, flash attention over
the cache, O product, fused residual add + norm, gate/up product, SwiGLU, down
product, residual add) against the same chain of oracle ops
(qw3lm_forward_batch, qwen3-lm.h:626-741).

Each op is held to its own bar in its own tests; here the chain is compared
end to end: the final hidden state within 2e-4 of its largest magnitude (the
products' fp32 roundings and the attention's 1e-4 * max|V| bar, passed through
two residual branches), and the cache slots written bit for bit except where a
rounding difference upstream moved a value across a Q8_0 rounding boundary
(at most one quantization step, in at most 1 % of the written elements)."""
import numpy as np
import pytest
from helpers import to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.qwen3 import Qwen3DecodeLayer, decode_mask

pytestmark = pytest.mark.gpu


def _w(r, n, k, s=0.05):
    return orc.quantize_q8_0((r.standard_normal((n, k)) * s).astype(np.float32))


@pytest.mark.parametrize("kv_type", ["q8_0", "f16"])
def test_decode_layer_matches_oracle_chain(dev, kv_type):
    print(f"qwen3 decode layer kv={kv_type}", flush=True)
    r = np.random.default_rng(31)
    H, Nh, Nkv, D, I, N, max_seq, n_sets, s0 = 256, 4, 2, 128, 512, 4, 512, 6, 1
    eps, theta = 1e-6, 1e6
    Wqkv, Wo, Wgu, Wd = _w(r, (Nh + 2 * Nkv) * D, H), _w(r, H, Nh * D), _w(r, 2 * I, H), _w(r, H, I)
    nw_in, nw_post = (1 + 0.1 * r.standard_normal(H)).astype(np.float32), (1 + 0.1 * r.standard_normal(H)).astype(
        np.float32)
    qn, kn = (1 + 0.1 * r.standard_normal(D)).astype(np.float32), (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    layer = Qwen3DecodeLayer(ops.Q8(to_dev(Wqkv)), ops.Q8(to_dev(Wo)), ops.Q8(to_dev(Wgu)), ops.Q8(to_dev(Wd)),
                             to_dev(nw_in), to_dev(nw_post), to_dev(qn), to_dev(kn), H, Nh, Nkv, D, I, max_seq,
                             n_sets, kv_type, eps, theta)
    # earlier tokens already in the caches (random but finite), then this step's
    pos = np.array([0, 37, 200, 255], np.int32)
    read_len = 256
    kc0 = (r.standard_normal((n_sets, Nkv, max_seq, D)) * 0.5).astype(np.float32)
    vc0 = (r.standard_normal((n_sets, Nkv, max_seq, D)) * 0.5).astype(np.float32)
    if kv_type == "q8_0":
        kq, vq = orc.quantize_q8_0(kc0, "x86"), orc.quantize_q8_0(vc0, "x86")
        layer.k_cache = ops.Q8(to_dev(kq))
        layer.v_cache = ops.Q8(to_dev(vq))
        kcache, vcache = orc.dequantize_q8_0(kq), orc.dequantize_q8_0(vq)
    else:
        kh, vh = orc.f32_to_f16(kc0), orc.f32_to_f16(vc0)
        layer.k_cache, layer.v_cache = to_dev(kh, f16=True), to_dev(vh, f16=True)
        kcache, vcache = orc.f16_to_f32(kh), orc.f16_to_f32(vh)
    hidden = (r.standard_normal((N, H)) * 0.8).astype(np.float32)
    sets = np.arange(s0, s0 + N, dtype=np.int32)
    y = to_np(layer.forward(to_dev(hidden), to_dev(pos), to_dev(sets), s0, read_len, decode_mask(pos, read_len)))

    # the oracle chain
    norm = orc.rms_norm_mul(hidden, nw_in, eps)
    qkv = orc.mul_mat_q8_0(Wqkv, norm)
    q = qkv[:, :Nh * D].reshape(N, Nh, D)
    k = qkv[:, Nh * D:(Nh + Nkv) * D].reshape(N, Nkv, D)
    v = qkv[:, (Nh + Nkv) * D:].reshape(N, Nkv, D)
    qo = orc.qk_norm_rope(q, qn, pos, eps, D, theta)
    ko = orc.qk_norm_rope(k, kn, pos, eps, D, theta)
    if kv_type == "q8_0":
        kw, vw = orc.dequantize_q8_0(orc.quantize_q8_0(ko, "x86")), orc.dequantize_q8_0(orc.quantize_q8_0(v, "x86"))
    else:
        kw, vw = orc.f16_to_f32(orc.f32_to_f16(ko)), orc.f16_to_f32(orc.f32_to_f16(v))
    for i in range(N):
        kcache[s0 + i, :, pos[i]] = kw[i]
        vcache[s0 + i, :, pos[i]] = vw[i]
    mask = np.where(np.arange(read_len)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
    attn = orc.flash_attn_ext(qo.reshape(N, Nh, 1, D), kcache[s0:s0 + N, :, :read_len],
                              vcache[s0:s0 + N, :, :read_len], mask.reshape(N, 1, 1, read_len), 1.0 / np.sqrt(D),
                              kv_type)
    o = orc.mul_mat_q8_0(Wo, attn.reshape(N, Nh * D))
    h1 = orc.add(hidden, o)
    n2 = orc.rms_norm_mul(h1, nw_post, eps)
    ref = orc.add(h1, orc.mul_mat_q8_0(Wd, orc.swiglu(orc.mul_mat_q8_0(Wgu, n2))))

    assert np.all(np.isfinite(y))
    assert np.max(np.abs(y - ref)) <= 2e-4 * np.max(np.abs(ref)), np.max(np.abs(y - ref))
    # the written cache slots
    if kv_type == "q8_0":
        kdev = orc.dequantize_q8_0(to_np(layer.k_cache.data))
        vdev = orc.dequantize_q8_0(to_np(layer.v_cache.data))
    else:
        kdev, vdev = orc.f16_to_f32(to_np(layer.k_cache)), orc.f16_to_f32(to_np(layer.v_cache))
    for i in range(N):
        for got, want in ((kdev[s0 + i, :, pos[i]], kw[i]), (vdev[s0 + i, :, pos[i]], vw[i])):
            diff = got != want
            assert diff.mean() <= 0.01
            if diff.any():
                step = np.max(np.abs(want)) / 127 * 1.01 if kv_type == "q8_0" else np.max(np.abs(want)) * 2 ** -10
                assert np.max(np.abs(got - want)) <= step
    # untouched slots keep their contents
    assert np.array_equal(kdev[0], kcache[0]) and np.array_equal(vdev[0], vcache[0])
