"""A whole Qwen3 prefill layer on the device (acestep_ops.qwen3.Qwen3Layer.prefill:
norm, Q8_0 QKV product, QK-norm + rope, K/V cache store of the new tokens,
flash attention over the cache under the causal mask, O product, fused residual
add + norm, gate/up product, SwiGLU, down product, residual add) against the
oracle, stage by stage (qw3lm_forward, qwen3-lm.h:429-549, with
qw3lm_build_attn, 330-424), for two sequences with earlier tokens already in
their cache sets (one starts at slot 0), at a small size and at the Qwen3-4B
layer shape (H 2560, 32/8 heads x 128, I 9728).

Every stage is checked against the oracle applied to the device's own inputs
of that stage, at that op's own bar:
  norm -> QKV product            Q8_0 product bound (the x quantization exact)
  QK-norm -> rope (q)            1e-5, row floor
  cache slots of the new tokens  bit-exact: Q8_0 (or fp16) of the roped K
                                 (recomputed by mi_qk_norm_rope on the layer's
                                 QKV buffer, which the fused launch equals) and V
  earlier slots, other sets      unchanged
  attention                      the kernels' derived bound (tests/fa_bound.py):
                                 the matrix-core prefill kernel (over an F16
                                 cache P in two 16-bit parts; over Q8_0 exact
                                 int8 block dots and V held as bf16 + f16 parts)
  O product, gate/up, down       Q8_0 product bound
  residual sums                  bit-exact (clamped to +-65504 with clamp_fp16)
With clamp_fp16 (qwen3-lm.h:53) the layer clamps V before the cache store
(qwen3-lm.h:392-393) and both residual sums (480-481, 488-489): the case drives V
and the hidden state past the fp16 range."""
import numpy as np
import pytest
from fa_bound import fa_bound
from helpers import assert_f32_close, assert_mul_mat_q8_0, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.qwen3 import Qwen3Layer

pytestmark = pytest.mark.gpu
LIM = 65504.0


def _w(r, n, k, s=0.05):
    return orc.quantize_q8_0((r.standard_normal((n, k)) * s).astype(np.float32))


# (H, Nh, Nkv, D, I, S new tokens, kv_pos per sequence, max_seq, n_sets, s0)
SIZES = {"small": (256, 4, 2, 128, 512, 37, (0, 100), 256, 4, 1),
         "qwen3_4b": (2560, 32, 8, 128, 9728, 96, (0, 300), 512, 3, 1)}


@pytest.mark.parametrize("size,kv_type,clamp", [("small", "f16", False), ("small", "q8_0", False),
                                                ("small", "q8_0", True), ("qwen3_4b", "f16", False),
                                                ("qwen3_4b", "q8_0", False)])
def test_prefill_layer_stage_by_stage(dev, size, kv_type, clamp):
    print(f"qwen3 prefill layer {size} kv={kv_type} clamp_fp16={clamp}", flush=True)
    r = np.random.default_rng(47)
    H, Nh, Nkv, D, I, S, kv_pos, max_seq, n_sets, s0 = SIZES[size]
    N = len(kv_pos)
    kv_pos = np.asarray(kv_pos, np.int64)
    eps, theta = 1e-6, 1e6
    Wqkv, Wo, Wgu, Wd = _w(r, (Nh + 2 * Nkv) * D, H), _w(r, H, Nh * D), _w(r, 2 * I, H), _w(r, H, I)
    nw_in = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)
    nw_post = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)
    qn, kn = (1 + 0.1 * r.standard_normal(D)).astype(np.float32), (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    hidden = (r.standard_normal((N, S, H)) * 0.8).astype(np.float32)
    if clamp:
        # V of most tokens past the fp16 range (the cache gets it clamped, qwen3-lm.h:392-393), and
        # residual sums past it (qwen3-lm.h:480-481, 488-489). Element 3 is fixed so that its
        # normalized value (at most ~7.1e6) stays below 127 * 65504, where the Q8_0 block scale of x
        # would overflow fp16 (in ggml as here).
        nw_in[3] = 2.5e6
        hidden[:, :, 3] = 2.0
        hidden[0, 0, :3] = [7e4, -9e4, 6e4]
    layer = Qwen3Layer(ops.Q8(to_dev(Wqkv)), ops.Q8(to_dev(Wo)), ops.Q8(to_dev(Wgu)), ops.Q8(to_dev(Wd)),
                       to_dev(nw_in), to_dev(nw_post), to_dev(qn), to_dev(kn), H, Nh, Nkv, D, I, max_seq, n_sets,
                       kv_type, eps, theta, clamp_fp16=clamp)
    # earlier tokens of each sequence (and every other slot) already hold finite values
    kc0 = r.standard_normal((n_sets, Nkv, max_seq, D), dtype=np.float32) * np.float32(0.5)
    vc0 = r.standard_normal((n_sets, Nkv, max_seq, D), dtype=np.float32) * np.float32(0.5)
    if kv_type == "q8_0":
        kq0, vq0 = orc.quantize_q8_0(kc0, "x86"), orc.quantize_q8_0(vc0, "x86")
        layer.k_cache, layer.v_cache = ops.Q8(to_dev(kq0)), ops.Q8(to_dev(vq0))
    else:
        kq0, vq0 = orc.f32_to_f16(kc0), orc.f32_to_f16(vc0)
        layer.k_cache, layer.v_cache = to_dev(kq0, f16=True), to_dev(vq0, f16=True)
    y = to_np(layer.prefill(to_dev(hidden), kv_pos, s0))
    b = {k: to_np(v) for k, v in layer._bufs.items() if not k.startswith("ws")}
    T = N * S
    h2 = hidden.reshape(T, H)
    pos = (kv_pos[:, None] + np.arange(S)[None, :]).astype(np.int32).reshape(T)

    # 1. input norm -> QKV product (one call)
    qkv = b["qkv"]
    assert_mul_mat_q8_0(qkv, Wqkv, orc.rms_norm_mul(h2, nw_in, eps))
    # 2. QK-norm -> rope: q from the layer's buffer; the roped K (which the fused
    # launch sends only to the cache) recomputed on the same QKV buffer
    q = qkv[:, :Nh * D].reshape(T, Nh, D)
    k = qkv[:, Nh * D:(Nh + Nkv) * D].reshape(T, Nkv, D)
    v = qkv[:, (Nh + Nkv) * D:].reshape(T, Nkv, D)
    dq = layer._bufs["qkv"]
    _, ko = ops.qk_norm_rope(dq[:, :Nh * D].unflatten(1, (Nh, D)), to_dev(qn), to_dev(pos), eps, D, theta,
                             k=dq[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D)), k_w=to_dev(kn))
    ko = to_np(ko)
    assert_f32_close(b["qo"], orc.qk_norm_rope(q, qn, pos, eps, D, theta), row_floor=True)
    assert_f32_close(ko, orc.qk_norm_rope(k, kn, pos, eps, D, theta), row_floor=True)
    if clamp:
        assert (np.abs(v) > LIM).sum() > v.size // 4
        v = orc.clamp(v, -LIM, LIM)
    # 3. the cache: the new tokens' slots bit-exact, every other slot unchanged
    if kv_type == "q8_0":
        kdev, vdev = to_np(layer.k_cache.data), to_np(layer.v_cache.data)
        kw, vw = orc.quantize_q8_0(ko, "x86"), orc.quantize_q8_0(v, "x86")
        kcache, vcache = orc.dequantize_q8_0(kdev), orc.dequantize_q8_0(vdev)
    else:
        kdev, vdev = to_np(layer.k_cache), to_np(layer.v_cache)
        kw, vw = orc.f32_to_f16(ko), orc.f32_to_f16(v)
        kcache, vcache = orc.f16_to_f32(kdev), orc.f16_to_f32(vdev)
    kexp, vexp = kq0.copy(), vq0.copy()
    for i in range(N):
        sl = slice(int(kv_pos[i]), int(kv_pos[i]) + S)
        kexp[s0 + i, :, sl] = kw[i * S:(i + 1) * S].transpose(1, 0, 2)
        vexp[s0 + i, :, sl] = vw[i * S:(i + 1) * S].transpose(1, 0, 2)
    assert np.array_equal(kdev, kexp)
    assert np.array_equal(vdev, vexp)
    # 4. attention over the device's cache under the causal mask, with the device's q
    kv_len = int((kv_pos + S).max())
    lim = kv_pos[:, None] + np.arange(S)[None, :]
    mask = np.where(np.arange(kv_len)[None, None, :] <= lim[:, :, None], 0.0, -np.inf).astype(np.float32)
    mask = mask.reshape(N, 1, S, kv_len)
    qf = np.ascontiguousarray(b["qo"].reshape(N, S, Nh, D).transpose(0, 2, 1, 3))
    kr, vr = kcache[s0:s0 + N, :, :kv_len], vcache[s0:s0 + N, :, :kv_len]
    attn = b["attn"]
    ref = orc.flash_attn_ext(qf, kr, vr, mask, 1.0 / np.sqrt(D), kv_type)
    mfma = "prefill" if S * (Nh // Nkv) >= 64 else False
    bound = fa_bound(qf, kr, vr, mask, 1.0 / np.sqrt(D), kv_type, mfma=mfma)
    assert np.all(np.isfinite(attn))
    assert np.all(np.abs(attn - ref) <= bound)
    # 5. O product; the residual sum (clamped with clamp_fp16) bit-exact
    a2 = attn.reshape(T, Nh * D)
    assert_mul_mat_q8_0(b["ao"], Wo, a2)
    h1 = orc.add_clamp(h2, b["ao"]) if clamp else orc.add(h2, b["ao"])
    assert np.array_equal(b["h1"], h1)
    # 6. post-attention norm -> gate/up product
    if clamp:
        assert_f32_close(b["n2"], orc.rms_norm_mul(h1, nw_post, eps))
        assert_mul_mat_q8_0(b["gu"], Wgu, b["n2"])
    else:
        assert_mul_mat_q8_0(b["gu"], Wgu, orc.rms_norm_mul(h1, nw_post, eps))
    # 7. SwiGLU -> down product; the last residual sum bit-exact (the layer adds h1
    # inside the down product's call, bit-identical to the product then the add)
    # the SwiGLU prologue quantizes the device's silu(g)*u (within ~1 ulp of the
    # oracle's, and bit-identical to mi_swiglu): the product is checked on those values
    mlp = to_np(ops.mul_mat_q8_0_swiglu(layer.w["down"], layer._bufs["gu"]))
    sw = to_np(ops.swiglu(layer._bufs["gu"]))
    assert_f32_close(sw, orc.swiglu(b["gu"]))
    assert_mul_mat_q8_0(mlp, Wd, sw)
    out = orc.add_clamp(h1, mlp) if clamp else orc.add(h1, mlp)
    assert np.array_equal(y.reshape(T, H), out)
    assert np.all(np.isfinite(y))


def test_prefill_rejects_slots_past_the_cache(dev):
    """kv_pos + S beyond max_seq is refused before any launch."""
    r = np.random.default_rng(5)
    H, Nh, Nkv, D, I = 256, 4, 2, 128, 512
    ws = [ops.Q8(to_dev(_w(r, n, k))) for n, k in (((Nh + 2 * Nkv) * D, H), (H, Nh * D), (2 * I, H), (H, I))]
    ones = lambda n: to_dev(np.ones(n, np.float32))  # noqa: E731
    layer = Qwen3Layer(*ws, ones(H), ones(H), ones(D), ones(D), H, Nh, Nkv, D, I, 64, 2, "f16")
    with pytest.raises(ValueError):
        layer.prefill(to_dev(np.zeros((1, 16, H), np.float32)), [60], 0)


@pytest.mark.parametrize("kv_type", ["f16", "q8_0"])
def test_prefill_layer_full_size_sampled(dev, kv_type):
    """The layer at the Qwen3-4B batched-prefill size: 2 sequences x 2048 new tokens
    (4096 rows through every product: the norm prologues take their 8-rows-per-
    workgroup form), one from slot 0 and one after 1000 cached tokens, 4096-slot
    caches. Every cache byte and both residual sums are checked in full (bit-exact);
    the products, QK-norm -> rope and attention on 40 sampled tokens (both
    sequences, both ends, tile edges) at the bars of the stage-by-stage test."""
    print(f"qwen3 prefill layer full size kv={kv_type}", flush=True)
    r = np.random.default_rng(53)
    H, Nh, Nkv, D, I = 2560, 32, 8, 128, 9728
    S, max_seq, n_sets, s0 = 2048, 4096, 2, 0
    kv_pos = np.asarray((0, 1000), np.int64)
    N = len(kv_pos)
    eps, theta = 1e-6, 1e6
    Wqkv, Wo, Wgu, Wd = _w(r, (Nh + 2 * Nkv) * D, H), _w(r, H, Nh * D), _w(r, 2 * I, H), _w(r, H, I)
    nw_in = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)
    nw_post = (1 + 0.1 * r.standard_normal(H)).astype(np.float32)
    qn, kn = (1 + 0.1 * r.standard_normal(D)).astype(np.float32), (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    hidden = (r.standard_normal((N, S, H)) * 0.8).astype(np.float32)
    layer = Qwen3Layer(ops.Q8(to_dev(Wqkv)), ops.Q8(to_dev(Wo)), ops.Q8(to_dev(Wgu)), ops.Q8(to_dev(Wd)),
                       to_dev(nw_in), to_dev(nw_post), to_dev(qn), to_dev(kn), H, Nh, Nkv, D, I, max_seq, n_sets,
                       kv_type, eps, theta)
    kc0 = r.standard_normal((n_sets, Nkv, max_seq, D), dtype=np.float32) * np.float32(0.5)
    vc0 = r.standard_normal((n_sets, Nkv, max_seq, D), dtype=np.float32) * np.float32(0.5)
    if kv_type == "q8_0":
        kq0, vq0 = orc.quantize_q8_0(kc0, "x86"), orc.quantize_q8_0(vc0, "x86")
        layer.k_cache, layer.v_cache = ops.Q8(to_dev(kq0)), ops.Q8(to_dev(vq0))
    else:
        kq0, vq0 = orc.f32_to_f16(kc0), orc.f32_to_f16(vc0)
        layer.k_cache, layer.v_cache = to_dev(kq0, f16=True), to_dev(vq0, f16=True)
    y = to_np(layer.prefill(to_dev(hidden), kv_pos, s0))
    b = {k: to_np(v) for k, v in layer._bufs.items() if not k.startswith("ws")}
    T = N * S
    h2 = hidden.reshape(T, H)
    pos = (kv_pos[:, None] + np.arange(S)[None, :]).astype(np.int32).reshape(T)
    tok = np.unique(np.r_[0, 1, 63, 64, 1023, 2046, 2047, 2048, 2049, 2111, 2112, 3071, 4094, 4095,
                          r.integers(0, T, 26)])

    # the products and QK-norm -> rope on the sampled tokens
    qkv = b["qkv"]
    assert_mul_mat_q8_0(qkv[tok], Wqkv, orc.rms_norm_mul(h2[tok], nw_in, eps))
    q = qkv[:, :Nh * D].reshape(T, Nh, D)
    k = qkv[:, Nh * D:(Nh + Nkv) * D].reshape(T, Nkv, D)
    v = qkv[:, (Nh + Nkv) * D:].reshape(T, Nkv, D)
    assert_f32_close(b["qo"][tok], orc.qk_norm_rope(q[tok], qn, pos[tok], eps, D, theta), row_floor=True)
    dq = layer._bufs["qkv"]
    _, ko = ops.qk_norm_rope(dq[:, :Nh * D].unflatten(1, (Nh, D)), to_dev(qn), to_dev(pos), eps, D, theta,
                             k=dq[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D)), k_w=to_dev(kn))
    ko = to_np(ko)
    assert_f32_close(ko[tok], orc.qk_norm_rope(k[tok], kn, pos[tok], eps, D, theta), row_floor=True)
    # every cache byte
    if kv_type == "q8_0":
        kdev, vdev = to_np(layer.k_cache.data), to_np(layer.v_cache.data)
        kw, vw = orc.quantize_q8_0(ko, "x86"), orc.quantize_q8_0(v, "x86")
        kcache, vcache = orc.dequantize_q8_0(kdev), orc.dequantize_q8_0(vdev)
    else:
        kdev, vdev = to_np(layer.k_cache), to_np(layer.v_cache)
        kw, vw = orc.f32_to_f16(ko), orc.f32_to_f16(v)
        kcache, vcache = orc.f16_to_f32(kdev), orc.f16_to_f32(vdev)
    kexp, vexp = kq0.copy(), vq0.copy()
    for i in range(N):
        sl = slice(int(kv_pos[i]), int(kv_pos[i]) + S)
        kexp[s0 + i, :, sl] = kw[i * S:(i + 1) * S].transpose(1, 0, 2)
        vexp[s0 + i, :, sl] = vw[i * S:(i + 1) * S].transpose(1, 0, 2)
    assert np.array_equal(kdev, kexp)
    assert np.array_equal(vdev, vexp)
    # attention of the sampled tokens over the device's cache under the causal mask
    kv_len = int((kv_pos + S).max())
    attn = b["attn"].reshape(N, S, Nh, D)
    for i in range(N):
        ts = tok[(tok >= i * S) & (tok < (i + 1) * S)] - i * S
        lim = kv_pos[i] + ts
        mask = np.where(np.arange(kv_len)[None, :] <= lim[:, None], 0.0, -np.inf).astype(np.float32)[None, None]
        qf = np.ascontiguousarray(b["qo"].reshape(N, S, Nh, D)[i:i + 1, ts].transpose(0, 2, 1, 3))
        kr, vr = kcache[s0 + i:s0 + i + 1, :, :kv_len], vcache[s0 + i:s0 + i + 1, :, :kv_len]
        ref = orc.flash_attn_ext(qf, kr, vr, mask, 1.0 / np.sqrt(D), kv_type)
        bound = fa_bound(qf, kr, vr, mask, 1.0 / np.sqrt(D), kv_type, mfma="prefill")
        got = attn[i:i + 1, ts]
        assert np.all(np.isfinite(got))
        assert np.all(np.abs(got - ref) <= bound)
    # O product (sampled); the residual sums in full, bit-exact
    assert_mul_mat_q8_0(b["ao"][tok], Wo, b["attn"].reshape(T, Nh * D)[tok])
    h1 = orc.add(h2, b["ao"])
    assert np.array_equal(b["h1"], h1)
    assert_mul_mat_q8_0(b["gu"][tok], Wgu, orc.rms_norm_mul(h1[tok], nw_post, eps))
    mlp = to_np(ops.mul_mat_q8_0_swiglu(layer.w["down"], layer._bufs["gu"]))
    sw = to_np(ops.swiglu(layer._bufs["gu"]))[tok]
    assert_f32_close(sw, orc.swiglu(b["gu"][tok]))
    assert_mul_mat_q8_0(mlp[tok], Wd, sw)
    assert np.array_equal(y.reshape(T, H), orc.add(h1, mlp))
