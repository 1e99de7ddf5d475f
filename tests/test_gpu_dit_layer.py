"""A whole ACE-Step DiT layer on the device (acestep_ops.dit.DiTLayer: AdaLN
norm -> modulate inside the Q8_0 QKV product, QK-norm + rope, F16 casts, flash
attention under the sliding-window or padding mask, O product, gated residual
and the next norm inside the next product, the cross attention over encoder states, the MLP with the
SwiGLU inside the down product, the last gated residual) against the oracle,
stage by stage (dit_ggml_build_layer, dit-graph.h:367-448), at a small size and
at the DiT's layer shape (H 2048, 16/8 heads x 128, I 6144).

Every stage is checked against the oracle applied to the device's own inputs
of that stage, at that op's own bar:
  QK-norm -> rope, the cross-attention per-head norms             1e-5 (row floor
                                                                 where values cancel)
  Q8_0 products (QKV, O, cross Q, cross K/V, gate/up, down)      Q8_0 product bound
                                                                 (those fed by a fused
                                                                 norm on the oracle's
                                                                 normalized rows)
  F16 casts of K and V                                           bit-exact
  attention                                                      the matrix-core
                                                                 kernel's derived bound
  gated and plain residual sums                                  bit-exact"""
import numpy as np
import pytest
from fa_bound import fa_bound
from helpers import assert_f32_close, assert_mul_mat_q8_0, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.device import DTensor
from acestep_ops.dit import DiTLayer

pytestmark = pytest.mark.gpu


def _w(r, n, k, s=0.05):
    return orc.quantize_q8_0((r.standard_normal((n, k)) * s).astype(np.float32))


def _f16_mask(m):
    return DTensor.from_numpy(np.ascontiguousarray(m.astype(np.float16)).view(np.uint16), "f16")


# (H, Nh, Nkv, D, I, S, N, enc_S)
SIZES = {"small": (256, 4, 2, 128, 512, 70, 2, 40), "dit": (2048, 16, 8, 128, 6144, 96, 2, 40)}


@pytest.mark.parametrize("size,cross,window", [("small", False, 32), ("small", True, 32), ("dit", True, 0),
                                               ("dit", False, 64)])
def test_dit_layer_stage_by_stage(dev, size, cross, window):
    print(f"dit layer {size} cross={cross} window={window}", flush=True)
    r = np.random.default_rng(59)
    H, Nh, Nkv, D, I, S, N, E = SIZES[size]
    eps, theta = 1e-6, 1e6
    T = N * S
    W = {"sa_qkv": _w(r, (Nh + 2 * Nkv) * D, H), "sa_o": _w(r, H, Nh * D), "gu": _w(r, 2 * I, H),
         "down": _w(r, H, I), "ca_q": _w(r, Nh * D, H), "ca_kv": _w(r, 2 * Nkv * D, H), "ca_o": _w(r, H, Nh * D)}
    nw = {k: (1 + 0.1 * r.standard_normal(n)).astype(np.float32)
          for k, n in (("sa", H), ("mlp", H), ("ca", H), ("qn", D), ("kn", D), ("cqn", D), ("ckn", D))}
    adaln = (0.3 * r.standard_normal((6, H))).astype(np.float32)
    shift_sa, scale_sa, gate_sa, shift_ff, scale_ff, gate_ff = adaln
    hidden = (r.standard_normal((N, S, H)) * 0.8).astype(np.float32)
    enc = (r.standard_normal((N, E, H)) * 0.8).astype(np.float32)
    ii = np.arange(S)
    # the self-attention mask: a sliding window (window > 0), else all zero (no padding)
    sa_m = np.where(np.abs(ii[None, :] - ii[:, None]) <= window, 0.0, -np.inf) if window else np.zeros((S, S))
    sa_m = np.ascontiguousarray(np.broadcast_to(sa_m, (N, 1, S, S))).astype(np.float32)
    # the cross-attention mask: sequence 1's last 7 encoder positions are padding
    ca_m = np.zeros((N, 1, S, E), np.float32)
    ca_m[1, :, :, E - 7:] = -np.inf
    q8 = lambda a: ops.Q8(to_dev(a))  # noqa: E731
    layer = DiTLayer(q8(W["sa_qkv"]), q8(W["sa_o"]), q8(W["gu"]), q8(W["down"]), to_dev(nw["sa"]), to_dev(nw["mlp"]),
                     to_dev(nw["qn"]), to_dev(nw["kn"]), H, Nh, Nkv, D, I, eps, theta,
                     **({"w_ca_q": q8(W["ca_q"]), "w_ca_kv": q8(W["ca_kv"]), "w_ca_o": q8(W["ca_o"]),
                         "ca_norm_w": to_dev(nw["ca"]), "ca_q_norm_w": to_dev(nw["cqn"]),
                         "ca_k_norm_w": to_dev(nw["ckn"])} if cross else {}))
    pos = np.tile(np.arange(S, dtype=np.int32), N)
    y = to_np(layer.forward(to_dev(hidden), to_dev(adaln), DiTLayer.positions(N, S), sa_mask=_f16_mask(sa_m),
                            enc=to_dev(enc) if cross else None, ca_mask=_f16_mask(ca_m) if cross else None))
    b = {k: to_np(v) for k, v in layer._bufs.items() if isinstance(k, str) and not k.startswith("ws")}
    h2 = hidden.reshape(T, H)
    scale = 1.0 / np.sqrt(D)
    mfma = "prefill" if S * (Nh // Nkv) >= 64 else False

    def attention(name, qo, k16, v16, n_kv, mask):
        qf = np.ascontiguousarray(qo.reshape(N, S, Nh, D).transpose(0, 2, 1, 3))
        kr = np.ascontiguousarray(orc.f16_to_f32(k16).reshape(N, n_kv, Nkv, D).transpose(0, 2, 1, 3))
        vr = np.ascontiguousarray(orc.f16_to_f32(v16).reshape(N, n_kv, Nkv, D).transpose(0, 2, 1, 3))
        ref = orc.flash_attn_ext(qf, kr, vr, mask, scale, "f16")
        bound = fa_bound(qf, kr, vr, mask, scale, "f16", mfma=mfma)
        got = b[name].reshape(N, S, Nh, D)  # y (N, S, Nh, D), as the oracle's
        assert np.all(np.isfinite(got)), name
        assert np.all(np.abs(got - ref) <= bound), name

    # 1. norm -> modulate -> the QKV product (one call: the normalized rows are made
    # inside the quantization of x, with the arithmetic of mi_rms_norm_modulate)
    qkv = b["qkv"]
    assert_mul_mat_q8_0(qkv, W["sa_qkv"], orc.rms_norm_modulate(h2, nw["sa"], scale_sa, shift_sa, eps))
    # 2. QK-norm -> rope; the F16 casts of K and V bit-exact
    q = qkv[:, :Nh * D].reshape(T, Nh, D)
    k = qkv[:, Nh * D:(Nh + Nkv) * D].reshape(T, Nkv, D)
    v = qkv[:, (Nh + Nkv) * D:].reshape(T, Nkv, D)
    # (the roped K, which the fused launch sends only to its F16 copy, recomputed by
    # mi_qk_norm_rope on the layer's QKV buffer: the fused launch equals it bit for bit)
    dq = layer._bufs["qkv"]
    _, ko = ops.qk_norm_rope(dq[:, :Nh * D].unflatten(1, (Nh, D)), to_dev(nw["qn"]), to_dev(pos), eps, D, theta,
                             k=dq[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D)), k_w=to_dev(nw["kn"]))
    ko = to_np(ko)
    assert_f32_close(b["qo"], orc.qk_norm_rope(q, nw["qn"], pos, eps, D, theta), row_floor=True)
    assert_f32_close(ko, orc.qk_norm_rope(k, nw["kn"], pos, eps, D, theta), row_floor=True)
    # K and V in F16, (N, Nkv, S, D)
    to_kv = lambda a: a.reshape(N, S, Nkv, D).transpose(0, 2, 1, 3)  # noqa: E731
    assert np.array_equal(b["k16"], to_kv(orc.f32_to_f16(ko)))
    assert np.array_equal(b["v16"], to_kv(orc.f32_to_f16(v)))
    # 3. self attention under its mask; the O product
    attention("attn", b["qo"], np.ascontiguousarray(b["k16"].transpose(0, 2, 1, 3)),
              np.ascontiguousarray(b["v16"].transpose(0, 2, 1, 3)), S, sa_m)
    assert_mul_mat_q8_0(b["sa_out"], W["sa_o"], b["attn"].reshape(T, Nh * D))
    if cross:
        # 4. the gated residual (bit-exact), the cross-attention norm and the cross Q
        # product (one call)
        h1 = orc.gated_add(h2, b["sa_out"], gate_sa)
        assert np.array_equal(b["h1"], h1)
        assert_mul_mat_q8_0(b["ca_q"], W["ca_q"], orc.rms_norm_mul(h1, nw["ca"], eps))
        # 5. K/V from the encoder states; the per-head norms; the F16 casts;
        # attention under the padding mask
        assert_mul_mat_q8_0(b["ca_kv"], W["ca_kv"], enc.reshape(N * E, H))
        kv = b["ca_kv"]
        assert_f32_close(b["ca_qn"], orc.rms_norm_mul(b["ca_q"].reshape(T, Nh, D), nw["cqn"], eps))
        assert_f32_close(b["ca_kn"], orc.rms_norm_mul(kv[:, :Nkv * D].reshape(N * E, Nkv, D), nw["ckn"], eps))
        assert np.array_equal(b["ca_k16"], orc.f32_to_f16(b["ca_kn"]))
        assert np.array_equal(b["ca_v16"], orc.f32_to_f16(kv[:, Nkv * D:].reshape(N * E, Nkv, D)))
        attention("ca_attn", b["ca_qn"], b["ca_k16"], b["ca_v16"], E, ca_m)
        assert_mul_mat_q8_0(b["ca_out"], W["ca_o"], b["ca_attn"].reshape(T, Nh * D))
        # 6. the plain residual (bit-exact)
        hf = orc.add(h1, b["ca_out"])
    else:
        hf = orc.gated_add(h2, b["sa_out"], gate_sa)
    assert np.array_equal(b["h2"], hf)
    # 7. the FFN norm -> modulate -> gate/up (one call); the down product (recomputed
    # by mi_mul_mat_q8_0_swiglu, which the layer's fused call equals before its gated
    # add) on the device's SwiGLU values (the prologue quantizes silu(g)*u as mi_swiglu
    # computes it, within ~1 ulp of the oracle's)
    assert_mul_mat_q8_0(b["gu"], W["gu"], orc.rms_norm_modulate(hf, nw["mlp"], scale_ff, shift_ff, eps))
    sw = to_np(ops.swiglu(layer._bufs["gu"]))
    assert_f32_close(sw, orc.swiglu(b["gu"]))
    mlp = to_np(ops.mul_mat_q8_0_swiglu(layer.w["down"], layer._bufs["gu"]))
    assert_mul_mat_q8_0(mlp, W["down"], sw)
    # 8. the last gated residual, bit-exact
    assert np.array_equal(y.reshape(T, H), orc.gated_add(hf, mlp, gate_ff))
    assert np.all(np.isfinite(y))


def test_dit_layer_encoder_kv_once(dev):
    """The cross attention's K and V computed once (DiTLayer.encode) and reused over two
    steps give the same layer outputs, bit for bit, as recomputing them from the
    encoder states in each step."""
    print("dit layer encoder K/V once", flush=True)
    r = np.random.default_rng(61)
    H, Nh, Nkv, D, I, S, N, E = SIZES["small"]
    q8 = lambda a: ops.Q8(to_dev(a))  # noqa: E731
    nw = lambda n: to_dev((1 + 0.1 * r.standard_normal(n)).astype(np.float32))  # noqa: E731
    layer = DiTLayer(q8(_w(r, (Nh + 2 * Nkv) * D, H)), q8(_w(r, H, Nh * D)), q8(_w(r, 2 * I, H)), q8(_w(r, H, I)),
                     nw(H), nw(H), nw(D), nw(D), H, Nh, Nkv, D, I, w_ca_q=q8(_w(r, Nh * D, H)),
                     w_ca_kv=q8(_w(r, 2 * Nkv * D, H)), w_ca_o=q8(_w(r, H, Nh * D)), ca_norm_w=nw(H),
                     ca_q_norm_w=nw(D), ca_k_norm_w=nw(D))
    enc = to_dev((r.standard_normal((N, E, H)) * 0.8).astype(np.float32))
    ca_m = np.zeros((N, 1, S, E), np.float32)
    ca_m[0, :, :, E - 5:] = -np.inf
    cmask = _f16_mask(ca_m)
    pos = DiTLayer.positions(N, S)
    adaln = to_dev((0.3 * r.standard_normal((6, H))).astype(np.float32))
    steps = [to_dev((r.standard_normal((N, S, H)) * 0.8).astype(np.float32)) for _ in range(2)]
    ref = [to_np(layer.forward(h, adaln, pos, enc=enc, ca_mask=cmask)) for h in steps]
    kv = layer.encode(enc)
    for h, y_ref in zip(steps, ref):
        y = to_np(layer.forward(h, adaln, pos, ca_mask=cmask, enc_kv=kv))
        assert np.array_equal(y, y_ref)
    with pytest.raises(ValueError):
        layer.forward(steps[0], adaln, pos, enc=enc, ca_mask=cmask, enc_kv=kv)


def test_dit_layer_rejects_cross_mismatch(dev):
    """enc must be given exactly when the layer holds cross-attention weights."""
    r = np.random.default_rng(3)
    H, Nh, Nkv, D, I = 256, 4, 2, 128, 512
    q8 = lambda a: ops.Q8(to_dev(a))  # noqa: E731
    ones = lambda n: to_dev(np.ones(n, np.float32))  # noqa: E731
    layer = DiTLayer(q8(_w(r, (Nh + 2 * Nkv) * D, H)), q8(_w(r, H, Nh * D)), q8(_w(r, 2 * I, H)), q8(_w(r, H, I)),
                     ones(H), ones(H), ones(D), ones(D), H, Nh, Nkv, D, I)
    h = to_dev(np.zeros((1, 8, H), np.float32))
    with pytest.raises(ValueError):
        layer.forward(h, to_dev(np.zeros((6, H), np.float32)), DiTLayer.positions(1, 8),
                      enc=to_dev(np.zeros((1, 4, H), np.float32)))
    with pytest.raises(ValueError):
        DiTLayer(q8(_w(r, (Nh + 2 * Nkv) * D, H)), q8(_w(r, H, Nh * D)), q8(_w(r, 2 * I, H)), q8(_w(r, H, I)),
                 ones(H), ones(H), ones(D), ones(D), H, Nh, Nkv, D, I, w_ca_q=q8(_w(r, Nh * D, H)))
