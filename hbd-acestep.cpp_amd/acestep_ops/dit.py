"""One ACE-Step DiT layer, every op on the device, with Q8_0 weights and F32
activations (dit_ggml_build_layer, dit-graph.h:367-448, with the self-attention
of dit_ggml_build_self_attn, 136-245, the cross attention of
dit_ggml_build_cross_attn, 274-354, and the MLP of dit_ggml_build_mlp, 249-268):

  norm_sa  = modulate(rms_norm(hidden) * sa_norm, scale_sa, shift_sa)  (404-405)
  qkv      = mul_mat(W_sa_qkv, norm_sa); q, k, v = views of qkv       (159-163)
  q, k     = rope(rms_norm(q|k) * q_norm|k_norm), positions 0..S-1     (181-198)
  k, v     = F16 casts                                                 (221-228)
  attn     = flash_attn_ext(q, k, v, sa_mask, 1/sqrt(D)), F32 precision (230-234)
  hidden   = hidden + mul_mat(W_sa_o, attn) * gate_sa                  (243, 415)
  cross attention (with encoder states enc):
    norm_ca = rms_norm(hidden) * ca_norm                               (424)
    q       = mul_mat(W_ca_q, norm_ca); k, v = views of mul_mat(W_ca_kv, enc)  (302-307)
    q, k    = rms_norm(q|k) * ca_q_norm|ca_k_norm (no rope)           (326-330)
    attn    = flash_attn_ext(q, F16 k, F16 v, ca_mask, 1/sqrt(D))     (334-348)
    hidden  = hidden + mul_mat(W_ca_o, attn)                          (353, 427)
  norm_ffn = modulate(rms_norm(hidden) * mlp_norm, scale_ffn, shift_ffn)  (437-438)
  hidden   = hidden + mul_mat(W_down, swiglu(mul_mat(W_gate_up, norm_ffn))) * gate_ffn  (439-440)

Each norm (with the gated or plain residual add before it and the modulate
after it) runs inside the quantization of the next product's x
(mi_mul_mat_q8_0_adaln: the normalized rows never go to memory), and the
SwiGLU inside the quantization of the down product's x with the last gated
residual where its outputs are formed (mi_mul_mat_q8_0_swiglu_gated_add); QK-norm -> rope writes K and V as F16 in the same
launch (mi_qk_norm_rope_kv_store). The six AdaLN vectors come in as one F32
(6, H) tensor: scale_shift_table + the timestep projection (dit-graph.h:384-399),
rows shift_sa, scale_sa, gate_sa, shift_ffn, scale_ffn, gate_ffn.

Shapes outermost first: hidden (N, S, H) F32; enc (N, enc_S, H) F32; sa_mask
(N, 1, S, S) F16 or None; ca_mask (N, 1, S, enc_S) F16 or None."""
from __future__ import annotations

import math

import numpy as np

from . import ops
from .device import DTensor


class DiTLayer:
    def __init__(self, w_sa_qkv, w_sa_o, w_gate_up, w_down, sa_norm_w, mlp_norm_w, sa_q_norm_w, sa_k_norm_w,
                 H: int, Nh: int, Nkv: int, D: int, I: int, eps: float = 1e-6, rope_theta: float = 1e6,
                 w_ca_q=None, w_ca_kv=None, w_ca_o=None, ca_norm_w=None, ca_q_norm_w=None, ca_k_norm_w=None,
                 stream=None):
        """w_*: Q8 weights in the GGUF layout (repacked here once); norms: F32 DTensors.
        The cross-attention weights are all given or all None."""
        self.H, self.Nh, self.Nkv, self.D, self.I = H, Nh, Nkv, D, I
        self.eps, self.theta, self.stream = eps, rope_theta, stream
        ws = {"sa_qkv": w_sa_qkv, "sa_o": w_sa_o, "gu": w_gate_up, "down": w_down}
        ca = (w_ca_q, w_ca_kv, w_ca_o, ca_norm_w, ca_q_norm_w, ca_k_norm_w)
        if any(x is not None for x in ca) and any(x is None for x in ca):
            raise ValueError("cross attention: give every weight or none")
        self.cross = w_ca_q is not None
        if self.cross:
            ws.update({"ca_q": w_ca_q, "ca_kv": w_ca_kv, "ca_o": w_ca_o})
        self.w = {name: ops.q8_0_repack(w, stream=stream) for name, w in ws.items()}
        self.sa_norm_w, self.mlp_norm_w = sa_norm_w, mlp_norm_w
        self.sa_q_norm_w, self.sa_k_norm_w = sa_q_norm_w, sa_k_norm_w
        self.ca_norm_w, self.ca_q_norm_w, self.ca_k_norm_w = ca_norm_w, ca_q_norm_w, ca_k_norm_w
        self._bufs = {}

    def _buf(self, name, shape, dtype="f32"):
        b = self._bufs.get(name)
        if b is None or b.shape != tuple(shape):
            b = DTensor.empty(tuple(shape), dtype)
            self._bufs[name] = b
        return b

    def _ws(self, name, x):
        need = ops.mul_mat_q8_0_workspace(self.w[name], x)
        return self._buf("ws_" + name, (max(need, 1),), "u8")

    def _fa(self, name, q, k, v, mask, out):
        need = ops.flash_attn_workspace(q, k, v)
        ws = self._buf("ws_fa_" + name, (max(need, 1),), "u8")
        return ops.flash_attn_ext(q, k, v, mask, 1.0 / math.sqrt(self.D), out=out, workspace=ws, stream=self.stream)

    def _seq_inputs(self, N: int):
        """Each sequence's first slot (0) and set (its index), for the K/V store."""
        key = ("seq", N)
        if key not in self._bufs:
            self._bufs[key] = (DTensor.from_numpy(np.zeros(N, np.int32)), DTensor.from_numpy(np.arange(N, dtype=np.int32)))
        return self._bufs[key]

    @staticmethod
    def positions(N: int, S: int) -> DTensor:
        """The rope positions: 0..S-1 for each of the N sequences (dit-graph.h:186-195)."""
        return DTensor.from_numpy(np.tile(np.arange(S, dtype=np.int32), N))

    def encode(self, enc):
        """The cross attention's K and V of the encoder states enc (N, enc_S, H) F32: the
        fused K/V product, the per-head K norm and both F16 casts (dit-graph.h:302-307,
        326-330, 338-343), as (k16, v16), each (N, enc_S, Nkv, D) F16. The encoder states
        are the same for every sampler step, so a caller may compute these once per
        generation and pass them to forward as enc_kv (the reference recomputes them in
        every step's graph; the values are the same). The tensors are the layer's own
        buffers: the next encode overwrites them."""
        if not self.cross:
            raise ValueError("encode: the layer has no cross-attention weights")
        Nkv, D, H = self.Nkv, self.D, self.H
        st = self.stream
        N, E = enc.shape[0], enc.shape[1]
        e2 = enc.view(N * E, H)
        kvc = ops.mul_mat_q8_0(self.w["ca_kv"], e2, out=self._buf("ca_kv", (N * E, 2 * Nkv * D)),
                               workspace=self._ws("ca_kv", e2), stream=st)
        kn = ops.rms_norm(kvc[:, 0:Nkv * D].unflatten(1, (Nkv, D)), self.eps, w=self.ca_k_norm_w,
                          out=self._buf("ca_kn", (N * E, Nkv, D)), stream=st)
        k16 = ops.cpy(kn, self._buf("ca_k16", (N * E, Nkv, D), "f16"), stream=st)
        v16 = ops.cpy(kvc[:, Nkv * D:2 * Nkv * D].unflatten(1, (Nkv, D)), self._buf("ca_v16", (N * E, Nkv, D), "f16"),
                      stream=st)
        return k16.view(N, E, Nkv, D), v16.view(N, E, Nkv, D)

    def forward(self, hidden, adaln, pos, sa_mask=None, enc=None, ca_mask=None, out=None, enc_kv=None):
        """hidden (N, S, H) F32 -> new hidden (N, S, H); adaln (6, H) F32; pos from
        positions(N, S); for a layer with cross attention, the encoder states enc (N,
        enc_S, H) F32, or their K and V from encode() as enc_kv."""
        N, S, H = hidden.shape
        Nh, Nkv, D, I = self.Nh, self.Nkv, self.D, self.I
        st = self.stream
        if enc is not None and enc_kv is not None:
            raise ValueError("give enc or enc_kv, not both")
        if self.cross != (enc is not None or enc_kv is not None):
            raise ValueError("enc (or enc_kv) is given exactly when the layer has cross-attention weights")
        T = N * S
        h2 = hidden.view(T, H)
        shift_sa, scale_sa, gate_sa, shift_ffn, scale_ffn, gate_ffn = (adaln[i] for i in range(6))

        # self attention: norm -> modulate -> the QKV product in one call
        qkv_dim = (Nh + 2 * Nkv) * D
        qkv = ops.mul_mat_q8_0_adaln(self.w["sa_qkv"], h2, self.sa_norm_w, self.eps, scale=scale_sa, shift=shift_sa,
                                     out=self._buf("qkv", (T, qkv_dim)), workspace=self._ws("sa_qkv", h2), stream=st)
        q = qkv[:, 0:Nh * D].unflatten(1, (Nh, D))
        k = qkv[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D))
        v = qkv[:, (Nh + Nkv) * D:qkv_dim].unflatten(1, (Nkv, D))
        # QK-norm -> rope and the F16 casts of K and V in one launch: K and V go to
        # F16 tensors laid out as a KV cache, (N, Nkv, S, D) with sequence b's token t
        # at slot t of set b -- the (N, heads, S, D) order flash attention reads
        # (ggml's permute(x, 0, 2, 1, 3), dit-graph.h:206-208)
        k16, v16 = self._buf("k16", (N, Nkv, S, D), "f16"), self._buf("v16", (N, Nkv, S, D), "f16")
        qo = ops.qk_norm_rope_kv_store(q, self.sa_q_norm_w, k, self.sa_k_norm_w, v, pos, self.eps, D, self.theta,
                                       k16, v16, self._seq_inputs(N)[0], sets=self._seq_inputs(N)[1],
                                       q_out=self._buf("qo", (T, Nh, D)), stream=st)
        attn = self._fa("sa", qo.view(N, S, Nh, D).permute(0, 2, 1, 3), k16, v16, sa_mask,
                        self._buf("attn", (N, S, Nh, D)))
        sa_out = ops.mul_mat_q8_0(self.w["sa_o"], attn.view(T, Nh * D), out=self._buf("sa_out", (T, H)),
                                  workspace=self._ws("sa_o", attn.view(T, Nh * D)), stream=st)
        if self.cross:
            # the gated residual, the cross-attention norm and the cross Q product in one call
            h1, qc = ops.mul_mat_q8_0_adaln(self.w["ca_q"], h2, self.ca_norm_w, self.eps, b=sa_out, gate=gate_sa,
                                            out_sum=self._buf("h1", (T, H)), out=self._buf("ca_q", (T, Nh * D)),
                                            workspace=self._ws("ca_q", h2), stream=st)
            ca_out = self._cross(qc, enc_kv if enc_kv is not None else self.encode(enc), ca_mask, N, S)
            # the cross-attention residual, the FFN norm -> modulate and the gate/up product in one call
            h2b, gu = ops.mul_mat_q8_0_adaln(self.w["gu"], h1, self.mlp_norm_w, self.eps, b=ca_out, scale=scale_ffn,
                                             shift=shift_ffn, out_sum=self._buf("h2", (T, H)),
                                             out=self._buf("gu", (T, 2 * I)), workspace=self._ws("gu", h1), stream=st)
        else:
            # the gated residual, the FFN norm -> modulate and the gate/up product in one call
            h2b, gu = ops.mul_mat_q8_0_adaln(self.w["gu"], h2, self.mlp_norm_w, self.eps, b=sa_out, gate=gate_sa,
                                             scale=scale_ffn, shift=shift_ffn, out_sum=self._buf("h2", (T, H)),
                                             out=self._buf("gu", (T, 2 * I)), workspace=self._ws("gu", h2), stream=st)
        # the MLP: SwiGLU inside the down product's quantization, the gated residual
        # where the product's outputs are formed
        need = ops.mul_mat_q8_0_swiglu_workspace(self.w["down"], gu)
        y = out.view(T, H) if out is not None else self._buf("out", (T, H))
        ops.mul_mat_q8_0_swiglu_gated_add(self.w["down"], gu, h2b, gate_ffn, out=y,
                                          workspace=self._buf("ws_down", (max(need, 1),), "u8"), stream=st)
        return y.view(N, S, H)

    def _cross(self, qc, enc_kv, ca_mask, N: int, S: int):
        """Cross attention of the layer's rows (their Q product qc (T, Nh * D)) over the
        encoder K and V (from encode): its O product (T, H)."""
        Nh, Nkv, D, H = self.Nh, self.Nkv, self.D, self.H
        st = self.stream
        T = N * S
        k16, v16 = enc_kv
        E = k16.shape[1]
        if k16.shape != (N, E, Nkv, D) or v16.shape != (N, E, Nkv, D):
            raise ValueError(f"enc_kv: K and V (N={N}, enc_S, {Nkv}, {D}) F16")
        qn = ops.rms_norm(qc.unflatten(1, (Nh, D)), self.eps, w=self.ca_q_norm_w,
                          out=self._buf("ca_qn", (T, Nh, D)), stream=st)
        attn = self._fa("ca", qn.view(N, S, Nh, D).permute(0, 2, 1, 3), k16.permute(0, 2, 1, 3),
                        v16.permute(0, 2, 1, 3), ca_mask, self._buf("ca_attn", (N, S, Nh, D)))
        return ops.mul_mat_q8_0(self.w["ca_o"], attn.view(T, Nh * D), out=self._buf("ca_out", (T, H)),
                                workspace=self._ws("ca_o", attn.view(T, Nh * D)), stream=st)
