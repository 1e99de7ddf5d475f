"""One Qwen3 decoder layer for batched decode, every op on the device
(qw3lm_forward_batch, qwen3-lm.h:626-741), with Q8_0 weights and a Q8_0 or
F16 KV cache:

  norm   = rms_norm(hidden) * input_layernorm                    (630)
  qkv    = mul_mat(W_qkv, norm); q, k, v = views of qkv           (637-642;
           the norm and the product as one call, mul_mat_q8_0_rms_norm)
  q, k   = rope(rms_norm(q|k) * q_norm|k_norm)                    (659-667)
  cache  <- k, v at slot kv_pos of each sequence's set            (682-703)
  attn   = flash_attn_ext(q, K[:read_len], V[:read_len], mask, 1/sqrt(D))  (706-723)
  hidden = hidden + mul_mat(W_o, attn)                            (729-733)
  norm2  = rms_norm(hidden) * post_attention_layernorm            (736; the add, the norm and the
           gate/up product as one call, mul_mat_q8_0_add_rms_norm)
  hidden = hidden + mul_mat(W_down, swiglu(mul_mat(W_gate_up, norm2)))  (737-741;
           swiglu and the down product as one call, mul_mat_q8_0_swiglu)

With clamp_fp16 (qwen3-lm.h:53, set from the CLI at pipeline-lm.cpp:616) V is
clamped to the fp16 range before the cache store (674-677) and both residual
sums are clamped (730-733, 738-741); the post-attention sum is then its own
add + norm call ahead of the gate/up product, since the fused add + norm +
product call has no clamp.

Shapes outermost first: hidden (N, H) F32 for N sequences of one token; the
caches (n_sets, Nkv, max_seq, D) (ggml [D, max_seq, Nkv, n_sets]); sequence i
uses set s0 + i, writes at pos[i] and attends to read_len slots under a mask
(N, 1, 1, read_len) F16 that is 0 up to pos[i] and -inf after."""
from __future__ import annotations

import math

import numpy as np

from . import ops
from .device import DTensor

FP16_MAX = 65504.0


def decode_mask(pos, read_len: int) -> DTensor:
    """F16 (N, 1, 1, read_len): 0 for slots <= pos[i] (the token just written
    included), -inf after -- the batched decode mask (qwen3-lm.h:582-596)."""
    pos = np.asarray(pos)
    m = np.where(np.arange(read_len)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float16)
    return DTensor.from_numpy(m.reshape(len(pos), 1, 1, read_len).view(np.uint16), "f16")


class Qwen3DecodeLayer:
    def __init__(self, w_qkv, w_o, w_gate_up, w_down, in_norm_w, post_norm_w, q_norm_w, k_norm_w, H: int, Nh: int,
                 Nkv: int, D: int, I: int, max_seq: int, n_sets: int, kv_type: str = "q8_0", eps: float = 1e-6,
                 rope_theta: float = 1e6, clamp_fp16: bool = False, stream=None):
        """w_*: Q8 weights in the GGUF layout (repacked here once); norms: F32 DTensors."""
        self.H, self.Nh, self.Nkv, self.D, self.I = H, Nh, Nkv, D, I
        self.eps, self.theta, self.stream = eps, rope_theta, stream
        self.clamp_fp16 = bool(clamp_fp16)
        self.w = {name: ops.q8_0_repack(w, stream=stream)
                  for name, w in (("qkv", w_qkv), ("o", w_o), ("gu", w_gate_up), ("down", w_down))}
        self.in_norm_w, self.post_norm_w = in_norm_w, post_norm_w
        self.q_norm_w, self.k_norm_w = q_norm_w, k_norm_w
        self.kv_type = kv_type
        if kv_type == "q8_0":
            self.k_cache = ops.Q8(DTensor.zeros((n_sets, Nkv, max_seq, D // 32 * 34), "u8"))
            self.v_cache = ops.Q8(DTensor.zeros((n_sets, Nkv, max_seq, D // 32 * 34), "u8"))
        elif kv_type == "f16":
            self.k_cache = DTensor.zeros((n_sets, Nkv, max_seq, D), "f16")
            self.v_cache = DTensor.zeros((n_sets, Nkv, max_seq, D), "f16")
        else:
            raise ValueError("kv_type: q8_0 or f16")
        self._bufs = {}

    def _buf(self, name, shape, dtype="f32"):
        b = self._bufs.get(name)
        if b is None or b.shape != tuple(shape):
            b = DTensor.empty(tuple(shape), dtype)
            self._bufs[name] = b
        return b

    def _cache_view(self, c, s0, n, read_len):
        if isinstance(c, ops.Q8):
            return ops.Q8(c.data[s0:s0 + n, :, :read_len])
        return c[s0:s0 + n, :, :read_len]

    def forward(self, hidden, pos, sets, s0: int, read_len: int, mask, out=None):
        """hidden (N, H) F32 -> new hidden (N, H); pos, sets: (N,) I32 device tensors."""
        N, H, Nh, Nkv, D, I = hidden.shape[0], self.H, self.Nh, self.Nkv, self.D, self.I
        st = self.stream
        qkv_dim = (Nh + 2 * Nkv) * D
        # the input norm and the QKV product in one call: the normalized rows are
        # made inside the quantization of the product's x
        qkv = ops.mul_mat_q8_0_rms_norm(self.w["qkv"], hidden, self.in_norm_w, self.eps,
                                        out=self._buf("qkv", (N, qkv_dim)), workspace=self._ws("qkv", hidden),
                                        stream=st)
        q = qkv[:, 0:Nh * D].unflatten(1, (Nh, D))
        k = qkv[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D))
        v = qkv[:, (Nh + Nkv) * D:qkv_dim].unflatten(1, (Nkv, D))
        # QK-norm -> rope, the V clamp and the K/V cache store in one launch (the
        # new tokens' slots are their positions)
        qo = ops.qk_norm_rope_kv_store(q, self.q_norm_w, k, self.k_norm_w, v, pos, self.eps, D, self.theta,
                                       self.k_cache, self.v_cache, pos, sets=sets, clamp_v=self.clamp_fp16,
                                       q_out=self._buf("qo", (N, Nh, D)), stream=st)
        kv = self._cache_view(self.k_cache, s0, N, read_len)
        vv = self._cache_view(self.v_cache, s0, N, read_len)
        qf = qo.unflatten(1, (Nh, 1))
        attn = self._buf("attn", (N, 1, Nh, D))
        ws = self._fa_ws(qf, kv, vv)
        ops.flash_attn_ext(qf, kv, vv, mask, 1.0 / math.sqrt(D), out=attn, workspace=ws, stream=st)
        a2 = attn.view(N, Nh * D)
        ao = ops.mul_mat_q8_0(self.w["o"], a2, out=self._buf("ao", (N, H)), workspace=self._ws("o", a2), stream=st)
        if self.clamp_fp16:
            h1, n2 = ops.add_rms_norm(hidden, ao, self.eps, w=self.post_norm_w, clamp=(-FP16_MAX, FP16_MAX),
                                      out_sum=self._buf("h1", (N, H)), out_norm=self._buf("n2", (N, H)), stream=st)
            gu = ops.mul_mat_q8_0(self.w["gu"], n2, out=self._buf("gu", (N, 2 * I)), workspace=self._ws("gu", n2),
                                  stream=st)
        else:
            # the residual add, the post-attention norm and the gate/up product in one call
            h1, gu = ops.mul_mat_q8_0_add_rms_norm(self.w["gu"], hidden, ao, self.post_norm_w, self.eps,
                                                   out_sum=self._buf("h1", (N, H)), out=self._buf("gu", (N, 2 * I)),
                                                   workspace=self._ws("gu", hidden), stream=st)
        # swiglu, the down projection and the residual add in one call: the SwiGLU
        # values are made inside the quantization of the product's x, and h1 is
        # added (then clamped under clamp_fp16) where the product's sum is formed
        # (bit-identical to the three ops)
        y = out if out is not None else self._buf("out", (N, H))
        return ops.mul_mat_q8_0_swiglu_add(self.w["down"], gu, h1, clamp=(-FP16_MAX, FP16_MAX) if self.clamp_fp16 else None,
                                           out=y, workspace=self._ws_glu("down", gu), stream=st)

    def _ws(self, name, x):
        need = ops.mul_mat_q8_0_workspace(self.w[name], x)
        return self._buf("ws_" + name, (max(need, 1),), "u8")

    def _ws_glu(self, name, gu):
        need = ops.mul_mat_q8_0_swiglu_workspace(self.w[name], gu)
        return self._buf("ws_" + name, (max(need, 1),), "u8")

    def _fa_ws(self, q, k, v):
        need = ops.flash_attn_workspace(q, k, v)
        return self._buf("ws_fa", (max(need, 1),), "u8")
