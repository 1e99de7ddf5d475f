"""GPU side of the GGUF loader: raw uploads, F16/BF16 widened to F32
(gf_load_tensor_f32), row-fused QKV and gate/up (gf_load_qkv_fused /
gf_load_pair_fused, gguf-weights.h:270-352), and a fused Q8_0 QKV weight
loaded, repacked and multiplied against the oracle on the concatenated rows."""
import os
import sys

import numpy as np
import pytest
from helpers import to_dev, to_np
from oracle import oracle as orc

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gguf_writer as gw  # noqa: E402

from acestep_ops import ops  # noqa: E402
from acestep_ops.gguf import GGUFModel  # noqa: E402

pytestmark = pytest.mark.gpu


def _model(tmp_path):
    r = np.random.default_rng(21)
    H, NQ, NKV = 256, 192, 64
    q = orc.quantize_q8_0(r.standard_normal((NQ, H)).astype(np.float32))
    k = orc.quantize_q8_0(r.standard_normal((NKV, H)).astype(np.float32))
    v = orc.quantize_q8_0(r.standard_normal((NKV, H)).astype(np.float32))
    g = orc.f32_to_bf16(r.standard_normal((96, H)).astype(np.float32))
    u = orc.f32_to_bf16(r.standard_normal((96, H)).astype(np.float32))
    u16 = orc.f32_to_f16(r.standard_normal((96, H)).astype(np.float32))
    nw = orc.f32_to_bf16(r.standard_normal((H,)).astype(np.float32))
    nh = orc.f32_to_f16(r.standard_normal((H,)).astype(np.float32))
    nf = r.standard_normal((H,)).astype(np.float32)
    ts = [("q", 8, [H, NQ], q), ("k", 8, [H, NKV], k), ("v", 8, [H, NKV], v), ("gate", 30, [H, 96], g),
          ("up", 30, [H, 96], u), ("up16", 1, [H, 96], u16), ("norm_bf16", 30, [H], nw), ("norm_f16", 1, [H], nh),
          ("norm_f32", 0, [H], nf)]
    data, _ = gw.build([("acestep-dit.block_count", gw.U32, 1)], [(n, t, ne, a.tobytes()) for n, t, ne, a in ts],
                       alignment=64)
    p = tmp_path / "w.gguf"
    p.write_bytes(data)
    return str(p), dict((n, a) for n, _, _, a in ts)


def test_uploads(dev, tmp_path):
    print("gguf uploads", flush=True)
    path, A = _model(tmp_path)
    with GGUFModel(path) as g:
        assert np.array_equal(to_np(g.load_tensor("q").data), A["q"])
        assert np.array_equal(to_np(g.load_tensor("gate")), A["gate"])
        assert np.array_equal(to_np(g.load_tensor_f32("norm_bf16")), orc.bf16_to_f32(A["norm_bf16"]))
        assert np.array_equal(to_np(g.load_tensor_f32("norm_f16")), orc.f16_to_f32(A["norm_f16"]))
        assert np.array_equal(to_np(g.load_tensor_f32("norm_f32")), A["norm_f32"])
        qkv = g.load_qkv_fused("q", "k", "v")
        assert np.array_equal(to_np(qkv.data), np.concatenate([A["q"], A["k"], A["v"]]))
        gu = g.load_pair_fused("gate", "up")
        assert np.array_equal(to_np(gu), np.concatenate([A["gate"], A["up"]]))
        assert g.load_pair_fused("gate", "up16") is None  # types differ: loaded separately
        assert g.try_load_tensor("absent") is None


def test_fused_q8_0_qkv_through_mul_mat(dev, tmp_path):
    print("gguf fused qkv mul_mat", flush=True)
    path, A = _model(tmp_path)
    with GGUFModel(path) as g:
        qkv = g.load_qkv_fused("q", "k", "v")
    w = np.concatenate([A["q"], A["k"], A["v"]])
    wr = ops.q8_0_repack(qkv)
    x = np.random.default_rng(22).standard_normal((40, 256)).astype(np.float32)
    y = to_np(ops.mul_mat_q8_0(wr, to_dev(x)))
    ref = orc.mul_mat_q8_0(w, x)
    wf = orc.dequantize_q8_0(w).astype(np.float64)
    xf = orc.dequantize_q8_0(orc.quantize_q8_0(x, "x86")).astype(np.float64)
    bound = (256 / 32 + 8) * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T) + 1e-30
    assert np.all(np.abs(y - ref) <= bound)
