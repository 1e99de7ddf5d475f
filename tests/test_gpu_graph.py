"""HIP-graph capture of one DiT block's fused ops: every replay, with eager
work and synchronizations in between, must equal the eager result bit for
bit (the kernels record no memset nodes)."""
import numpy as np
import pytest

from helpers import randn, to_dev
from oracle import oracle as orc

from acestep_ops import device, ops
from acestep_ops.device import DTensor, Graph, Stream

pytestmark = pytest.mark.gpu


def test_dit_block_graph_replays_match_eager(dev):
    rows, H, nh, nkv, D, I = 256, 2048, 16, 8, 128, 6144
    bf = lambda a: to_dev(orc.f32_to_bf16(a), dev, bf16=True)  # noqa: E731
    hidden, sa_out, ffn_out = bf(randn((rows, H), 1)), bf(randn((rows, H), 2)), bf(randn((rows, H), 3))
    qkv = bf(randn((rows, (nh + 2 * nkv) * D), 4))
    gu = bf(randn((rows, 2 * I), 5))
    ad = to_dev(randn((6 * H,), 6, scale=0.1), dev)
    w1, w2 = to_dev(randn((H,), 7, 0.1, 1.0), dev), to_dev(randn((H,), 8, 0.1, 1.0), dev)
    qw = to_dev(randn((D,), 9, 0.1, 1.0), dev)
    pos = to_dev(np.arange(rows, dtype=np.int32), dev)
    v = [ad[i * H:(i + 1) * H] for i in range(6)]
    q = qkv[:, :nh * D].unflatten(1, (nh, D))
    k = qkv[:, nh * D:(nh + nkv) * D].unflatten(1, (nkv, D))
    outs = {n: DTensor.empty(s, "bf16") for n, s in
            [("norm_sa", (rows, H)), ("q", (rows, nh, D)), ("k", (rows, nkv, D)), ("h1", (rows, H)),
             ("norm_ff", (rows, H)), ("ff", (rows, I)), ("h2", (rows, H))]}
    st = Stream()

    def block():
        ops.rms_norm_modulate(hidden, w1, v[1], v[0], 1e-6, out=outs["norm_sa"], stream=st.handle)
        ops.qk_norm_rope(q, qw, pos, 1e-6, D, 1e4, k=k, k_w=qw, q_out=outs["q"], k_out=outs["k"], stream=st.handle)
        ops.add_rms_norm(hidden, sa_out, 1e-6, gate=v[2], w=w2, scale=v[4], shift=v[3], out_sum=outs["h1"],
                         out_norm=outs["norm_ff"], stream=st.handle)
        ops.swiglu(gu, out=outs["ff"], stream=st.handle)
        ops.gated_add(outs["h1"], ffn_out, v[5], out=outs["h2"], stream=st.handle)

    block()
    st.synchronize()
    eager = {n: t.numpy() for n, t in outs.items()}
    g = Graph()
    with g.capture(st):
        block()
    for rep in range(3):
        for t in outs.values():
            t.fill_byte(0x7F)  # scribble between replays
        ops.add(hidden, sa_out)  # unrelated eager work on the null stream
        device.synchronize()
        g.launch()
        st.synchronize()
        for n, t in outs.items():
            assert np.array_equal(t.numpy(), eager[n]), f"replay {rep}: {n} differs from eager"
