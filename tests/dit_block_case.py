"""One ACE-Step DiT block's inputs, descriptors and oracle, shared by the GPU
parity test of ``mi_dit_block_ops`` and the CPU audit of its descriptors.

The block follows dit_ggml_build_layer (dit-graph.h:367-448): H=2048,
16 Q / 8 KV heads x 128, SwiGLU I=6144, on S frames x N=2 (the CFG pair).
With ``cross`` the cross-attention branch is included (dit-graph.h:426-433):
its norm fused behind the self-attention residual, its Q-norm and K-norm on
the permuted per-head views the reference builds (dit-graph.h:317-331), and
the plain residual add fused with the FFN norm.

``mk`` supplies device storage: ``mk.empty(shape, dtype)`` and
``mk.up(array, dtype)``; the GPU test passes real allocations, the CPU audit
passes stand-ins that only record sizes.
"""
from __future__ import annotations

import numpy as np

from helpers import randn
from oracle import oracle as orc

EPS = 1e-6
H, NH, NKV, D, I, THETA = 2048, 16, 8, 128, 6144, 1e4


def build(dt: str, cross: bool, mk, S: int = 96, N: int = 2, enc_S: int = 40):
    """Returns (io, host, outs): the filled MiDitBlockIO, the host inputs (bf16
    bit patterns for bf16 activations) and the output views to read back."""
    from acestep_ops import _lib, ops

    bf16 = dt == "bf16"
    act = "bf16" if bf16 else "f32"
    R = S * N
    kv_dim = NKV * D
    cv = orc.f32_to_bf16 if bf16 else (lambda a: a)
    host = {
        "h": cv(randn((N, S, H), seed=1)),
        "ad": randn((6 * H,), seed=2, scale=0.1),
        "saw": randn((H,), seed=3, scale=0.1, mean=1.0),
        "ffw": randn((H,), seed=4, scale=0.1, mean=1.0),
        "qkv": cv(randn((N, S, (NH + 2 * NKV) * D), seed=5)),
        "sa_out": cv(randn((N, S, H), seed=6)),
        "gu": cv(randn((N, S, 2 * I), seed=7)),
        "ffn_out": cv(randn((N, S, H), seed=8)),
        "qw": randn((D,), seed=9, scale=0.1, mean=1.0),
        "kw": randn((D,), seed=10, scale=0.1, mean=1.0),
        "pos": np.tile(np.arange(S, dtype=np.int32), N),
    }
    if cross:
        host.update({
            "caw": randn((H,), seed=11, scale=0.1, mean=1.0),
            "ca_qlin": cv(randn((N, S, NH * D), seed=12)),        # q projection of norm_ca
            "ca_kv": cv(randn((N, enc_S, 2 * kv_dim), seed=13)),  # fused K+V projection of enc
            "ca_qw": randn((D,), seed=14, scale=0.1, mean=1.0),
            "ca_kw": randn((D,), seed=15, scale=0.1, mean=1.0),
            "ca_out": cv(randn((N, S, H), seed=16)),
        })
    dev = {k: mk.up(a, act if k in ACT_KEYS else None) for k, a in host.items()}
    qkv = dev["qkv"].view(R, -1)
    outs = {
        "norm_sa": mk.empty((N, S, H), act),
        "q_out": mk.empty((R, NH, D), act),
        "k_out": mk.empty((R, NKV, D), act),
        "norm_ffn": mk.empty((N, S, H), act),
        "ff": mk.empty((N, S, I), act),
        "hidden": dev["h"],
    }
    io = _lib.MiDitBlockIO()
    io.hidden, io.adaln = ops.desc(dev["h"]), ops.desc(dev["ad"])
    io.sa_norm_w, io.ffn_norm_w = ops.desc(dev["saw"]), ops.desc(dev["ffw"])
    io.norm_sa, io.norm_ffn = ops.desc(outs["norm_sa"]), ops.desc(outs["norm_ffn"])
    io.q = ops.desc(qkv[:, :NH * D].unflatten(1, (NH, D)))
    io.k = ops.desc(qkv[:, NH * D:(NH + NKV) * D].unflatten(1, (NKV, D)))
    io.q_w, io.k_w = ops.desc(dev["qw"]), ops.desc(dev["kw"])
    io.q_out, io.k_out, io.pos = ops.desc(outs["q_out"]), ops.desc(outs["k_out"]), ops.desc(dev["pos"])
    io.sa_out, io.gate_up = ops.desc(dev["sa_out"]), ops.desc(dev["gu"])
    io.ff, io.ffn_out = ops.desc(outs["ff"]), ops.desc(dev["ffn_out"])
    io.eps, io.rope_freq_base, io.n_dims, io.use_cross_attn = EPS, THETA, D, int(cross)
    if cross:
        outs["norm_ca"] = mk.empty((N, S, H), act)
        outs["ca_q_out"] = mk.empty((N, NH, S, D), act)     # ggml [D, S, Nh, N], contiguous
        outs["ca_k_out"] = mk.empty((N, NKV, enc_S, D), act)
        # q: [H, S, N] -> [D, Nh, S, N] -> permute -> [D, S, Nh, N] (dit-graph.h:317-318)
        ca_q = dev["ca_qlin"].unflatten(2, (NH, D)).permute(0, 2, 1, 3)
        # k: the first kv_dim columns of the fused K+V product, per head, permuted (319-320)
        ca_k = dev["ca_kv"][:, :, :kv_dim].unflatten(2, (NKV, D)).permute(0, 2, 1, 3)
        io.ca_norm_w, io.norm_ca = ops.desc(dev["caw"]), ops.desc(outs["norm_ca"])
        io.ca_q, io.ca_q_w, io.ca_q_out = ops.desc(ca_q), ops.desc(dev["ca_qw"]), ops.desc(outs["ca_q_out"])
        io.ca_k, io.ca_k_w, io.ca_k_out = ops.desc(ca_k), ops.desc(dev["ca_kw"]), ops.desc(outs["ca_k_out"])
        io.ca_out = ops.desc(dev["ca_out"])
    return io, host, outs, dev


ACT_KEYS = ("h", "qkv", "sa_out", "gu", "ffn_out", "ca_qlin", "ca_kv", "ca_out")


def reference(dt: str, cross: bool, host: dict, S: int = 96, N: int = 2, enc_S: int = 40) -> dict:
    """The unfused ggml node sequence of dit_ggml_build_layer on the oracle.
    For bf16 every node output the graph stores is rounded to bf16 before the
    next node reads it; returned arrays are bf16 bit patterns then."""
    bf16 = dt == "bf16"
    R = S * N
    kv_dim = NKV * D
    ch = (lambda fn, *a, **kw: orc.bf16_chain(fn, *a, **kw)) if bf16 else (lambda fn, *a, **kw: fn(*a, **kw))
    ad = host["ad"]
    shift_sa, scale_sa, gate_sa, shift_ff, scale_ff, gate_ff = (ad[i * H:(i + 1) * H] for i in range(6))
    h = host["h"].reshape(R, H)
    qkv = host["qkv"].reshape(R, -1)
    ref = {
        "norm_sa": ch(orc.rms_norm_modulate, h, host["saw"], scale_sa, shift_sa, EPS),
        "q_out": ch(orc.qk_norm_rope, qkv[:, :NH * D].reshape(R, NH, D), host["qw"], host["pos"], EPS, D, THETA),
        "k_out": ch(orc.qk_norm_rope, qkv[:, NH * D:(NH + NKV) * D].reshape(R, NKV, D), host["kw"], host["pos"],
                    EPS, D, THETA),
    }
    h1 = ch(orc.gated_add, h, host["sa_out"].reshape(R, H), gate_sa)
    if cross:
        ref["norm_ca"] = ch(orc.rms_norm_mul, h1, host["caw"], EPS)
        q = host["ca_qlin"].reshape(N, S, NH, D).transpose(0, 2, 1, 3)
        k = host["ca_kv"][:, :, :kv_dim].reshape(N, enc_S, NKV, D).transpose(0, 2, 1, 3)
        ref["ca_q_out"] = ch(orc.rms_norm_mul, np.ascontiguousarray(q), host["ca_qw"], EPS)
        ref["ca_k_out"] = ch(orc.rms_norm_mul, np.ascontiguousarray(k), host["ca_kw"], EPS)
        h1 = ch(orc.add, h1, host["ca_out"].reshape(R, H))
    ref["norm_ffn"] = ch(orc.rms_norm_modulate, h1, host["ffw"], scale_ff, shift_ff, EPS)
    ref["ff"] = ch(orc.swiglu, host["gu"].reshape(R, 2 * I))
    ref["hidden"] = ch(orc.gated_add, h1, host["ffn_out"].reshape(R, H), gate_ff)
    return ref


# outputs whose values are differences that can cancel (row-RMS floor applies)
ROW_FLOOR = {"norm_sa": True, "q_out": True, "k_out": True, "norm_ffn": True, "norm_ca": False,
             "ca_q_out": False, "ca_k_out": False, "ff": False, "hidden": True}
# outputs the library must reproduce bit for bit (sums rounded as the nodes store them)
BIT_EXACT = ("hidden",)
