"""GPU parity of the layer-chain drivers (one DiT block, one Qwen3 layer) and
of the timestep embedding, against the oracle's unfused ggml node sequence
in the reference builders' order."""
import ctypes

import numpy as np
import pytest

import dit_block_case
from helpers import assert_bf16_ulp, assert_f32_close, randn, rng, to_dev, to_np, tsembd_bar
from oracle import oracle as orc

from acestep_ops import _lib, device, ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu
EPS = 1e-6


def test_timestep_embedding(dev):
    t = (rng(1).uniform(0, 1, 64) * 1000).astype(np.float32)
    t[:3] = [0.0, 1000.0, 0.5]
    y = to_np(ops.timestep_embedding(to_dev(t, dev), 256, 10000))
    tsembd_bar(y, orc.timestep_embedding(t, 256, 10000), t, 256, 10000)
    y = to_np(ops.timestep_embedding(to_dev(t, dev), 7, 100))
    tsembd_bar(y, orc.timestep_embedding(t, 7, 100), t, 7, 100)
    assert not y[:, 6].any()


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_scale(dev, dt):
    """ggml_scale: y = x * s, one rounding (bit-exact); in place and on a strided view."""
    bf16 = dt == "bf16"
    x = randn((37, 300), seed=21) * 10
    x[0, :4] = [np.inf, -0.0, np.nan, 3e38]
    xh = orc.f32_to_bf16(x) if bf16 else x
    f = orc.bf16_to_f32 if bf16 else (lambda a: a)
    cv = orc.f32_to_bf16 if bf16 else (lambda a: a)
    d = to_dev(xh, dev, bf16=bf16)
    for s in (1000.0, -0.37, 2.0 ** -20):
        y = to_np(ops.scale(d, s))
        assert np.array_equal(y.view(np.uint8), cv(orc.scale(f(xh), s)).view(np.uint8)), s
    v = d[3:30:2, 7:263]  # rows at a stride, columns offset
    y = to_np(ops.scale(v, 1000.0))
    assert np.array_equal(y.view(np.uint8), cv(orc.scale(f(xh)[3:30:2, 7:263], 1000.0)).view(np.uint8))
    ops.scale(d, 0.5, out=d)
    assert np.array_equal(to_np(d).view(np.uint8), cv(orc.scale(f(xh), 0.5)).view(np.uint8))


def test_timestep_scale_then_embedding(dev):
    """The DiT's timestep path: t ~ U[0, 1] for the CFG pair's one graph, scaled by
    1000 (ggml_scale, dit-graph.h:87), then the 256-wide sinusoidal embedding (90)."""
    t = rng(5).uniform(0, 1, 1).astype(np.float32)
    ts = ops.scale(to_dev(t, dev), 1000.0)
    tsh = orc.scale(t, 1000.0)
    assert np.array_equal(to_np(ts).view(np.uint32), tsh.view(np.uint32))
    y = to_np(ops.timestep_embedding(ts, 256, 10000))
    tsembd_bar(y, orc.timestep_embedding(tsh, 256, 10000), tsh, 256, 10000)


class _DevStorage:
    """Device storage for the shared DiT block case."""

    @staticmethod
    def empty(shape, dtype):
        return DTensor.empty(shape, dtype)

    @staticmethod
    def up(a, dtype):
        return DTensor.from_numpy(a, dtype)


@pytest.mark.parametrize("cross", [False, True], ids=["self_only", "cross_attn"])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_dit_block_chain(dev, dt, cross):
    """ACE-Step DiT block (H=2048, 16/8 heads x 128, I=6144) on S=96 x N=2 rows,
    with and without the cross-attention branch (dit-graph.h:426-433), against
    the unfused node sequence. Every descriptor is checked against its
    allocation on the host first (ops.desc and test_chain_descriptors_cpu)."""
    print(f"dit block chain {dt} cross={cross}", flush=True)
    io, host, outs, _keep = dit_block_case.build(dt, cross, _DevStorage)
    _lib.call("mi_dit_block_ops", ctypes.byref(io), None)
    device.synchronize()
    refs = dit_block_case.reference(dt, cross, host)
    for name, r in refs.items():
        print("check", name, flush=True)
        got = to_np(outs[name]).reshape(r.shape)
        if name in dit_block_case.BIT_EXACT:
            assert np.array_equal(got, r), name
        elif dt == "bf16":
            assert_bf16_ulp(got, r, row_floor=dit_block_case.ROW_FLOOR[name])
        else:
            assert_f32_close(got, r, row_floor=dit_block_case.ROW_FLOOR[name])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_qwen3_layer_chain_decode(dev, dt):
    """Qwen3-4B-shaped decode step, batch 8, clamp_fp16 on, Q8_0 KV cache; F32
    and the bf16 activations of the batch-8 decode configuration."""
    print(f"qwen3 layer chain decode {dt}", flush=True)
    bf16 = dt == "bf16"
    H, nh, nkv, D, I, N, max_seq, theta = 2560, 32, 8, 128, 9728, 8, 8192, 1e6
    r = rng(3)
    h = randn((N, H), seed=1)
    h[0, :4] = [7e4, -7e4, 1e5, 3.0]
    qkv = randn((N, (nh + 2 * nkv) * D), seed=2)
    qkv[1, (nh + nkv) * D] = 9e4  # a V value beyond the fp16 range: clamped before the store
    attn_out = randn((N, H), seed=3)
    gu = randn((N, 2 * I), seed=4)
    mlp_out = randn((N, H), seed=5)
    w_in = randn((H,), seed=6, scale=0.1, mean=1.0)
    w_post = randn((H,), seed=7, scale=0.1, mean=1.0)
    qw = randn((D,), seed=8, scale=0.1, mean=1.0)
    kw = randn((D,), seed=9, scale=0.1, mean=1.0)
    pos = r.integers(0, max_seq, N).astype(np.int32)
    sets = np.arange(N, dtype=np.int32)
    act = "bf16" if bf16 else "f32"
    if bf16:
        h, qkv, attn_out, gu, mlp_out = (orc.f32_to_bf16(a) for a in (h, qkv, attn_out, gu, mlp_out))
    up = lambda a: DTensor.from_numpy(a, act)  # noqa: E731

    hd, qkvd = up(h), up(qkv)
    qd = qkvd[:, :nh * D].unflatten(1, (nh, D))
    kd = qkvd[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
    vd = qkvd[:, (nh + nkv) * D:].unflatten(1, (nkv, D))
    rb = D // 32 * 34
    kc = DTensor.zeros((N, nkv, max_seq, rb), "u8")
    vc = DTensor.zeros((N, nkv, max_seq, rb), "u8")
    norm = DTensor.empty((N, H), act)
    norm2 = DTensor.empty((N, H), act)
    q_out = DTensor.empty((N, nh, D), act)
    k_out = DTensor.empty((N, nkv, D), act)
    ff = DTensor.empty((N, I), act)
    err = DTensor.zeros((1,), "i32")
    keep = [to_dev(a, dev) for a in (w_in, w_post, qw, kw, pos, pos, sets)] + [up(a) for a in (attn_out, gu, mlp_out)]
    io = _lib.MiQwen3LayerIO()
    io.hidden, io.in_norm_w, io.post_norm_w = ops.desc(hd), ops.desc(keep[0]), ops.desc(keep[1])
    io.norm, io.norm2 = ops.desc(norm), ops.desc(norm2)
    io.q, io.k, io.v = ops.desc(qd), ops.desc(kd), ops.desc(vd)
    io.q_w, io.k_w, io.q_out, io.k_out, io.pos = (ops.desc(keep[2]), ops.desc(keep[3]), ops.desc(q_out),
                                                  ops.desc(k_out), ops.desc(keep[4]))
    io.k_cache, io.v_cache, io.pos0, io.sets = ops.desc(ops.Q8(kc)), ops.desc(ops.Q8(vc)), ops.desc(keep[5]), ops.desc(keep[6])
    io.attn_out, io.gate_up, io.ff, io.mlp_out = ops.desc(keep[7]), ops.desc(keep[8]), ops.desc(ff), ops.desc(keep[9])
    io.eps, io.rope_freq_base, io.n_dims, io.clamp_fp16, io.kv_rounding = EPS, theta, D, 1, _lib.Q8_0_CPU_X86
    io.d_err = err.ptr
    _lib.call("mi_qwen3_layer_ops", ctypes.byref(io), None)
    device.synchronize()

    # oracle: qw3lm_forward_batch node order (qwen3-lm.h:632-741); in bf16 each
    # stored node output is rounded to bf16 before the next node reads it
    ch = orc.bf16_chain if bf16 else (lambda fn, *a, **kw: fn(*a, **kw))
    f32 = orc.bf16_to_f32 if bf16 else (lambda a: a)
    n1 = ch(orc.rms_norm_mul, h, w_in, EPS)
    qh = qkv[:, :nh * D].reshape(N, nh, D)
    kh = qkv[:, nh * D:(nh + nkv) * D].reshape(N, nkv, D)
    vh = ch(orc.clamp, qkv[:, (nh + nkv) * D:].reshape(N, nkv, D), -65504.0, 65504.0)
    qo = ch(orc.qk_norm_rope, qh, qw, pos, EPS, D, theta)
    ko = ch(orc.qk_norm_rope, kh, kw, pos, EPS, D, theta)
    h1 = ch(orc.add_clamp, h, attn_out)
    n2 = ch(orc.rms_norm_mul, h1, w_post, EPS)
    ffr = ch(orc.swiglu, gu)
    h2 = ch(orc.add_clamp, h1, mlp_out)
    close = (lambda a, b, **kw: assert_bf16_ulp(a, b, **kw)) if bf16 else assert_f32_close
    close(to_np(norm), n1)
    close(to_np(q_out), qo, row_floor=True)
    close(to_np(k_out), ko, row_floor=True)
    assert np.array_equal(to_np(hd), h2)  # add + clamp is bit-exact
    close(to_np(norm2), n2)
    close(to_np(ff), ffr)
    assert int(err.item()) == 0
    kch, vch = to_np(kc), to_np(vc)
    kq = orc.quantize_q8_0(f32(to_np(k_out)), "x86")  # the store quantizes the kernel's own k_out
    vq = orc.quantize_q8_0(f32(vh), "x86")
    for b in range(N):
        assert np.array_equal(kch[b, :, pos[b]], kq[b])
        assert np.array_equal(vch[b, :, pos[b]], vq[b])


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_qwen3_layer_fused_kv_path(dev, dt):
    """The driver with k_out empty (QK-norm, rope, V clamp and KV store as one
    mi_qk_norm_rope_kv_store launch) against the driver with k_out (the three
    calls), same inputs: every output and both caches bit-identical; V is left
    as it was on the fused path."""
    print(f"qwen3 layer fused kv path {dt}", flush=True)
    H, nh, nkv, D, I, N, max_seq = 2560, 32, 8, 128, 9728, 8, 8192
    r = rng(5)
    act = dt
    mk = lambda a: DTensor.from_numpy(orc.f32_to_bf16(a), "bf16") if dt == "bf16" else DTensor.from_numpy(a)  # noqa
    qkv0 = randn((N, (nh + 2 * nkv) * D), seed=12)
    qkv0[2, (nh + nkv) * D + 5] = -9e4
    consts = [to_dev(a, dev) for a in (randn((H,), seed=16, scale=0.1, mean=1.0), randn((H,), seed=17, scale=0.1,
              mean=1.0), randn((D,), seed=18, scale=0.1, mean=1.0), randn((D,), seed=19, scale=0.1, mean=1.0),
              r.integers(0, max_seq, N).astype(np.int32), np.arange(N, dtype=np.int32))]
    ins = [mk(randn((N, H), seed=13)), mk(randn((N, 2 * I), seed=14)), mk(randn((N, H), seed=15))]
    res = []
    for fused in (False, True):
        hd, qkvd = mk(randn((N, H), seed=11)), mk(qkv0)
        qd = qkvd[:, :nh * D].unflatten(1, (nh, D))
        kd = qkvd[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
        vd = qkvd[:, (nh + nkv) * D:].unflatten(1, (nkv, D))
        rb = D // 32 * 34
        kc, vc = DTensor.zeros((N, nkv, max_seq, rb), "u8"), DTensor.zeros((N, nkv, max_seq, rb), "u8")
        outs = dict(norm=DTensor.empty((N, H), act), norm2=DTensor.empty((N, H), act),
                    q_out=DTensor.empty((N, nh, D), act), ff=DTensor.empty((N, I), act))
        k_out = DTensor.empty((N, nkv, D), act)
        io = _lib.MiQwen3LayerIO()
        io.hidden, io.in_norm_w, io.post_norm_w = ops.desc(hd), ops.desc(consts[0]), ops.desc(consts[1])
        io.norm, io.norm2 = ops.desc(outs["norm"]), ops.desc(outs["norm2"])
        io.q, io.k, io.v = ops.desc(qd), ops.desc(kd), ops.desc(vd)
        io.q_w, io.k_w, io.q_out, io.pos = (ops.desc(consts[2]), ops.desc(consts[3]), ops.desc(outs["q_out"]),
                                            ops.desc(consts[4]))
        if not fused:
            io.k_out = ops.desc(k_out)
        io.k_cache, io.v_cache = ops.desc(ops.Q8(kc)), ops.desc(ops.Q8(vc))
        io.pos0, io.sets = ops.desc(consts[4]), ops.desc(consts[5])
        io.attn_out, io.gate_up, io.ff, io.mlp_out = (ops.desc(ins[0]), ops.desc(ins[1]), ops.desc(outs["ff"]),
                                                      ops.desc(ins[2]))
        io.eps, io.rope_freq_base, io.n_dims, io.clamp_fp16, io.kv_rounding = EPS, 1e6, D, 1, _lib.Q8_0_CPU_X86
        _lib.call("mi_qwen3_layer_ops", ctypes.byref(io), None)
        device.synchronize()
        res.append({**{k: to_np(v) for k, v in outs.items()}, "hidden": to_np(hd), "kc": to_np(kc),
                    "vc": to_np(vc), "v": to_np(vd)})
    a, b = res
    for name in ("norm", "norm2", "q_out", "ff", "hidden", "kc", "vc"):
        assert np.array_equal(a[name], b[name]), name
    v0 = to_np(mk(qkv0)[:, (nh + nkv) * D:].unflatten(1, (nkv, D)))
    assert np.array_equal(b["v"], v0) and not np.array_equal(a["v"], v0)  # only the three calls clamp V in place
