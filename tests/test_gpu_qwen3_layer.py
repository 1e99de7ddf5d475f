"""A whole Qwen3 decode layer on the device (acestep_ops.qwen3.Qwen3DecodeLayer:
norm, Q8_0 QKV product, QK-norm + rope, KV-cache write, flash attention over
the cache, O product, fused residual add + norm, gate/up product, SwiGLU, down
product, residual add) against the oracle, stage by stage
(qw3lm_forward_batch, qwen3-lm.h:626-741), at a small size and at the
Qwen3-4B batch-8 decode shape (H 2560, 32/8 heads x 128, I 9728, 8192-slot
caches, positions up to 8191).

Every stage is checked against the oracle applied to the device's own inputs
of that stage (read back from the layer's buffers), at that op's own bar:
  norm -> QKV product            Q8_0 product bound (the x quantization exact)
  QK-norm -> rope                1e-5, row floor (the layer writes K only to the
                                 cache, in the same launch; the device's roped K
                                 is recomputed from its QKV buffer by
                                 mi_qk_norm_rope, which that launch equals)
  cache slots (K and V)          bit-exact: Q8_0 of the device's roped K and V,
                                 or their fp16 values
  attention                      the kernels' derived bound (tests/fa_bound.py)
  O product, gate/up, down       Q8_0 product bound
  residual sums                  bit-exact (clamped to +-65504 with clamp_fp16)
With clamp_fp16 (qwen3-lm.h:53) the layer clamps V before the cache store
(674-677; the QKV buffer keeps the product) and both residual sums (730-733,
738-741): the case drives V and the hidden state past the fp16 range."""
import numpy as np
import pytest
from fa_bound import fa_bound
from helpers import assert_f32_close, assert_mul_mat_q8_0, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.qwen3 import Qwen3DecodeLayer, decode_mask

pytestmark = pytest.mark.gpu
LIM = 65504.0


def _w(r, n, k, s=0.05):
    return orc.quantize_q8_0((r.standard_normal((n, k)) * s).astype(np.float32))


# (H, Nh, Nkv, D, I, N, max_seq, n_sets, s0): a small layer, and the
# Qwen3-4B decode layer at batch 8 over 8192-slot caches (one set more than
# the batch, so one set stays untouched)
SIZES = {"small": (256, 4, 2, 128, 512, 4, 512, 6, 1),
         "qwen3_4b_b8": (2560, 32, 8, 128, 9728, 8, 8192, 9, 1)}


@pytest.mark.parametrize("size,kv_type,clamp", [("small", "q8_0", False), ("small", "f16", False),
                                                ("small", "q8_0", True), ("qwen3_4b_b8", "q8_0", False),
                                                ("qwen3_4b_b8", "f16", False), ("qwen3_4b_b8", "q8_0", True)])
def test_decode_layer_stage_by_stage(dev, size, kv_type, clamp):
    print(f"qwen3 decode layer {size} kv={kv_type} clamp_fp16={clamp}", flush=True)
    r = np.random.default_rng(31)
    H, Nh, Nkv, D, I, N, max_seq, n_sets, s0 = SIZES[size]
    eps, theta = 1e-6, 1e6
    Wqkv, Wo, Wgu, Wd = _w(r, (Nh + 2 * Nkv) * D, H), _w(r, H, Nh * D), _w(r, 2 * I, H), _w(r, H, I)
    nw_in, nw_post = (1 + 0.1 * r.standard_normal(H)).astype(np.float32), (1 + 0.1 * r.standard_normal(H)).astype(
        np.float32)
    qn, kn = (1 + 0.1 * r.standard_normal(D)).astype(np.float32), (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    hidden = (r.standard_normal((N, H)) * 0.8).astype(np.float32)
    if clamp:
        # V of most tokens past the fp16 range; the normalized x stays below 127 * 65504,
        # where its Q8_0 block scale would overflow fp16 (in ggml as here)
        nw_in[3] = 4e6
        hidden[0, :3] = [7e4, -9e4, 6e4]    # residual sums past the fp16 range
    layer = Qwen3DecodeLayer(ops.Q8(to_dev(Wqkv)), ops.Q8(to_dev(Wo)), ops.Q8(to_dev(Wgu)), ops.Q8(to_dev(Wd)),
                             to_dev(nw_in), to_dev(nw_post), to_dev(qn), to_dev(kn), H, Nh, Nkv, D, I, max_seq,
                             n_sets, kv_type, eps, theta, clamp_fp16=clamp)
    # earlier tokens already in the caches (random but finite), then this step's
    if size == "small":
        pos = np.array([0, 37, 200, 255], np.int32)
    else:  # positions U[0, 8191] with the extremes included
        pos = np.concatenate([[0, max_seq - 1], r.integers(0, max_seq, N - 2)]).astype(np.int32)
    read_len = int(min(max_seq, (pos.max() + 1 + 255) // 256 * 256))  # the 256-bucketed read (qwen3-lm.h:582-596)
    kc0 = r.standard_normal((n_sets, Nkv, max_seq, D), dtype=np.float32) * np.float32(0.5)
    vc0 = r.standard_normal((n_sets, Nkv, max_seq, D), dtype=np.float32) * np.float32(0.5)
    if kv_type == "q8_0":
        kq, vq = orc.quantize_q8_0(kc0, "x86"), orc.quantize_q8_0(vc0, "x86")
        layer.k_cache, layer.v_cache = ops.Q8(to_dev(kq)), ops.Q8(to_dev(vq))
        kcache0 = orc.dequantize_q8_0(kq)
    else:
        kh, vh = orc.f32_to_f16(kc0), orc.f32_to_f16(vc0)
        layer.k_cache, layer.v_cache = to_dev(kh, f16=True), to_dev(vh, f16=True)
        kcache0 = orc.f16_to_f32(kh)
    sets = np.arange(s0, s0 + N, dtype=np.int32)
    y = to_np(layer.forward(to_dev(hidden), to_dev(pos), to_dev(sets), s0, read_len, decode_mask(pos, read_len)))
    b = {k: to_np(v) for k, v in layer._bufs.items() if not k.startswith("ws")}

    # 1. input norm -> QKV product (one call)
    qkv = b["qkv"]
    v_cols = slice((Nh + Nkv) * D, (Nh + 2 * Nkv) * D)
    norm = orc.rms_norm_mul(hidden, nw_in, eps)
    assert_mul_mat_q8_0(qkv, Wqkv, norm)
    # 2. QK-norm -> rope on the device's q, k. The layer writes K only to the
    # cache (one launch with the store, bit-identical to mi_qk_norm_rope then
    # mi_kv_store); the device's roped K is mi_qk_norm_rope on the same buffer.
    q = qkv[:, :Nh * D].reshape(N, Nh, D)
    k = qkv[:, Nh * D:(Nh + Nkv) * D].reshape(N, Nkv, D)
    v = qkv[:, v_cols].reshape(N, Nkv, D)
    dq = layer._bufs["qkv"]
    _, ko = ops.qk_norm_rope(dq[:, :Nh * D].unflatten(1, (Nh, D)), to_dev(qn), to_dev(pos), eps, D, theta,
                             k=dq[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D)), k_w=to_dev(kn))
    ko = to_np(ko)
    assert_f32_close(b["qo"], orc.qk_norm_rope(q, qn, pos, eps, D, theta), row_floor=True)
    assert_f32_close(ko, orc.qk_norm_rope(k, kn, pos, eps, D, theta), row_floor=True)
    if clamp:
        # V past the fp16 range for most tokens; the cache gets it clamped (674-677)
        assert (np.abs(v) > LIM).sum() > v.size // 4
        v = orc.clamp(v, -LIM, LIM)
    # 3. the written cache slots: the device's roped K and (clamped) V, bit-exact
    if kv_type == "q8_0":
        kdev = to_np(layer.k_cache.data)
        vdev = to_np(layer.v_cache.data)
        kw, vw = orc.quantize_q8_0(ko, "x86"), orc.quantize_q8_0(v, "x86")
        kcache, vcache = orc.dequantize_q8_0(kdev), orc.dequantize_q8_0(vdev)
    else:
        kdev, vdev = to_np(layer.k_cache), to_np(layer.v_cache)
        kw, vw = orc.f32_to_f16(ko), orc.f32_to_f16(v)
        kcache, vcache = orc.f16_to_f32(kdev), orc.f16_to_f32(vdev)
    for i in range(N):
        assert np.array_equal(kdev[s0 + i, :, pos[i]], kw[i])
        assert np.array_equal(vdev[s0 + i, :, pos[i]], vw[i])
    assert np.array_equal(kcache[0], kcache0[0])  # an untouched set keeps its contents
    # 4. attention over the device's cache, with the device's q
    mask = np.where(np.arange(read_len)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
    mask = mask.reshape(N, 1, 1, read_len)
    qf = b["qo"].reshape(N, Nh, 1, D)
    kr, vr = kcache[s0:s0 + N, :, :read_len], vcache[s0:s0 + N, :, :read_len]
    attn = b["attn"]
    ref = orc.flash_attn_ext(qf, kr, vr, mask, 1.0 / np.sqrt(D), kv_type)
    # every cache type runs a matrix-core decode kernel (P, or P times V's block
    # scale, in two 16-bit parts)
    bound = fa_bound(qf, kr, vr, mask, 1.0 / np.sqrt(D), kv_type, mfma=True)
    assert np.all(np.abs(attn - ref) <= bound)
    # 5. O product; the residual sum (clamped with clamp_fp16) bit-exact
    assert_mul_mat_q8_0(b["ao"], Wo, attn.reshape(N, Nh * D))
    h1 = orc.add_clamp(hidden, b["ao"]) if clamp else orc.add(hidden, b["ao"])
    assert np.array_equal(b["h1"], h1)
    # 6. post-attention norm -> gate/up product
    if clamp:
        assert_f32_close(b["n2"], orc.rms_norm_mul(h1, nw_post, eps))
        assert_mul_mat_q8_0(b["gu"], Wgu, b["n2"])
    else:
        assert_mul_mat_q8_0(b["gu"], Wgu, orc.rms_norm_mul(h1, nw_post, eps))
    # 7. SwiGLU -> down product; the last residual sum bit-exact. The layer adds
    # h1 inside the down product's call (mi_mul_mat_q8_0_swiglu_add), which equals
    # mi_mul_mat_q8_0_swiglu then the add: the device's product alone is that
    # call on the layer's own gate/up output
    mlp = to_np(ops.mul_mat_q8_0_swiglu(layer.w["down"], layer._bufs["gu"]))
    assert_mul_mat_q8_0(mlp, Wd, orc.swiglu(b["gu"]))
    out = orc.add_clamp(h1, mlp) if clamp else orc.add(h1, mlp)
    assert np.array_equal(y, out)
    assert np.all(np.isfinite(y))
