"""One Qwen3 decoder layer, every op on the device, with Q8_0 weights and a
Q8_0 or F16 KV cache: batched decode (Qwen3Layer.forward, qw3lm_forward_batch,
qwen3-lm.h:626-741) and prefill (Qwen3Layer.prefill, qw3lm_forward,
qwen3-lm.h:429-549 with qw3lm_build_attn, 330-424). Decode:

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
(N, 1, 1, read_len) F16 that is 0 up to pos[i] and -inf after.

Prefill runs the same node sequence over S new tokens of each of N sequences
(the reference runs one sequence per call; N > 1 batches several): the
products take the N * S rows at once, token t of sequence b has position
kv_pos[b] + t and is stored at that slot of set s0 + b (qwen3-lm.h:396-406),
and attention reads the first kv_len = max_b(kv_pos[b] + S) slots under the
causal mask (N, 1, S, kv_len) F16, 0 for slots <= kv_pos[b] + t and -inf
after (qwen3-lm.h:523-533): q (N, Nh, S, D) is a strided view of the roped q
rows, as ggml's permute makes it (qwen3-lm.h:380)."""
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


def causal_mask(kv_pos, S: int, kv_len: int) -> DTensor:
    """F16 (N, 1, S, kv_len): row t of sequence b is 0 for slots <= kv_pos[b] + t
    and -inf after -- the prefill mask (qwen3-lm.h:523-533) for each sequence."""
    kv_pos = np.asarray(kv_pos, np.int64)
    lim = kv_pos[:, None] + np.arange(S)[None, :]  # (N, S)
    m = np.where(np.arange(kv_len)[None, None, :] <= lim[:, :, None], 0.0, -np.inf).astype(np.float16)
    return DTensor.from_numpy(m.reshape(len(kv_pos), 1, S, kv_len).view(np.uint16), "f16")


class Qwen3Layer:
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
        N, Nh, Nkv, D = hidden.shape[0], self.Nh, self.Nkv, self.D
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
        return self._tail(hidden, attn.view(N, Nh * D), out)

    def prefill(self, hidden, kv_pos, s0: int, out=None):
        """hidden (N, S, H) F32 -> new hidden (N, S, H): S new tokens of each of N
        sequences; kv_pos (host ints, N): the slot of each sequence's first new
        token (its earlier tokens already in the cache); sequence b uses set s0 + b.
        prefill_inputs then prefill_run."""
        inp = self.prefill_inputs(kv_pos, hidden.shape[1], s0)
        self._inputs = inp  # alive until the next call: the launches read them
        return self.prefill_run(hidden, inp, out)

    def prefill_inputs(self, kv_pos, S: int, s0: int) -> dict:
        """The host-built inputs of a prefill step, uploaded (qwen3-lm.h:513-533):
        token positions, each sequence's first slot and set, the causal mask."""
        kv_pos = np.asarray(kv_pos, np.int64).reshape(-1)
        N = len(kv_pos)
        max_seq = self.k_cache.data.shape[2] if isinstance(self.k_cache, ops.Q8) else self.k_cache.shape[2]
        kv_len = int((kv_pos + S).max())
        if kv_pos.min() < 0 or kv_len > max_seq:
            raise ValueError(f"prefill: slots [kv_pos, kv_pos + {S}) must lie in [0, {max_seq})")
        return {"S": S, "s0": s0, "kv_len": kv_len,
                "pos": DTensor.from_numpy((kv_pos[:, None] + np.arange(S)[None, :]).astype(np.int32).reshape(N * S)),
                "pos0": DTensor.from_numpy(kv_pos.astype(np.int32)),
                "sets": DTensor.from_numpy(np.arange(s0, s0 + N, dtype=np.int32)),
                "mask": causal_mask(kv_pos, S, kv_len)}

    def prefill_run(self, hidden, inp: dict, out=None):
        """The launches of a prefill step (no host transfer: a graph may capture
        them) on hidden (N, S, H) with inputs from prefill_inputs."""
        N, S, H = hidden.shape
        Nh, Nkv, D = self.Nh, self.Nkv, self.D
        st = self.stream
        assert S == inp["S"] and N == inp["pos0"].shape[0]
        s0, kv_len, pos, pos0, sets, mask = inp["s0"], inp["kv_len"], inp["pos"], inp["pos0"], inp["sets"], inp["mask"]
        T = N * S
        h2 = hidden.view(T, H)
        qkv_dim = (Nh + 2 * Nkv) * D
        qkv = ops.mul_mat_q8_0_rms_norm(self.w["qkv"], h2, self.in_norm_w, self.eps,
                                        out=self._buf("qkv", (T, qkv_dim)), workspace=self._ws("qkv", h2), stream=st)
        q = qkv[:, 0:Nh * D].unflatten(1, (Nh, D))
        k = qkv[:, Nh * D:(Nh + Nkv) * D].unflatten(1, (Nkv, D))
        v = qkv[:, (Nh + Nkv) * D:qkv_dim].unflatten(1, (Nkv, D))
        # QK-norm -> rope, the V clamp and the cache store of all T tokens in one
        # launch (token t of the flat order is token t % S of sequence t / S)
        qo = ops.qk_norm_rope_kv_store(q, self.q_norm_w, k, self.k_norm_w, v, pos, self.eps, D, self.theta,
                                       self.k_cache, self.v_cache, pos0, sets=sets, clamp_v=self.clamp_fp16,
                                       q_out=self._buf("qo", (T, Nh, D)), stream=st)
        kv = self._cache_view(self.k_cache, s0, N, kv_len)
        vv = self._cache_view(self.v_cache, s0, N, kv_len)
        qf = qo.view(N, S, Nh, D).permute(0, 2, 1, 3)  # (N, Nh, S, D), ggml's permute(q, 0, 2, 1, 3)
        attn = self._buf("attn", (N, S, Nh, D))
        ws = self._fa_ws(qf, kv, vv)
        ops.flash_attn_ext(qf, kv, vv, mask, 1.0 / math.sqrt(D), out=attn, workspace=ws, stream=st)
        y = self._tail(h2, attn.view(T, Nh * D), None if out is None else out.view(T, H))
        return y.view(N, S, H)

    def _tail(self, hidden, a2, out):
        """The O product, the residual sums, the post-attention norm and the MLP on
        rows of hidden (rows, H) and attention output a2 (rows, Nh * D)."""
        N, H, I = hidden.shape[0], self.H, self.I
        st = self.stream
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


Qwen3DecodeLayer = Qwen3Layer  # the name the decode-only callers use
