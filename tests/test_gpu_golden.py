"""GPU parity against the committed golden fixtures (tests/golden/*.npz).

Each fixture holds seeded inputs with edge cases and the oracle's outputs;
the HIP path is checked at this path's bars: Q8_0 and the elementwise
add / gated add / clamp bit-exact, fp32 <= 1e-5 relative (row-RMS floor where
outputs are differences that can cancel), bf16 within 1 ulp.
"""
import os

import numpy as np
import pytest

from helpers import GOLDEN, assert_bf16_ulp, assert_f32_close, to_dev, to_np, tsembd_bar

from acestep_ops import ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu


def _fx(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def test_golden_rms_norm_modulate_f32(dev):
    f = _fx("rms_norm_modulate_f32")
    x, w, eps = to_dev(f["x"]), to_dev(f["w"]), float(f["eps"])
    assert_f32_close(to_np(ops.rms_norm(x, eps, w)), f["y_norm"])
    y = ops.rms_norm_modulate(x, w, to_dev(f["scale"]), to_dev(f["shift"]), eps)
    assert_f32_close(to_np(y), f["y_mod"], row_floor=True)


def test_golden_dit_bf16(dev):
    f = _fx("dit_bf16")
    h, x = to_dev(f["h"], bf16=True), to_dev(f["x"], bf16=True)
    w, sc, sh, g = (to_dev(f[k]) for k in ("w", "scale", "shift", "gate"))
    eps = float(f["eps"])
    assert_bf16_ulp(to_np(ops.rms_norm_modulate(h, w, sc, sh, eps)), f["y_mod"], row_floor=True)
    assert np.array_equal(to_np(ops.gated_add(h, x, g)), f["y_sum"])
    ys, yn = ops.add_rms_norm(h, x, eps, gate=g, w=w, scale=sc, shift=sh)
    assert np.array_equal(to_np(ys), f["y_sum"])
    assert_bf16_ulp(to_np(yn), f["y_sum_norm"], row_floor=True)


@pytest.mark.parametrize("name", ["qk_rope_f32", "qk_rope_bf16"])
def test_golden_qk_norm_rope(dev, name):
    f = _fx(name)
    bf = name.endswith("bf16")
    q, k = to_dev(f["q"], bf16=bf), to_dev(f["k"], bf16=bf)
    qo, ko = ops.qk_norm_rope(q, to_dev(f["q_w"]), to_dev(f["pos"]), float(f["eps"]), 128, float(f["theta"]),
                              k=k, k_w=to_dev(f["k_w"]))
    for got, ref in ((qo, f["q_out"]), (ko, f["k_out"])):
        if bf:
            assert_bf16_ulp(to_np(got), ref, row_floor=True)
        else:
            assert_f32_close(to_np(got), ref, row_floor=True)


def test_golden_swiglu_f32(dev):
    f = _fx("swiglu_f32")
    gu = to_dev(f["gu"])
    assert_f32_close(to_np(ops.swiglu(gu)), f["y"])
    assert_f32_close(to_np(ops.swiglu(gu, swapped=True)), f["y_swapped"])


def test_golden_add_clamp_f32(dev):
    f = _fx("add_clamp_f32")
    y = to_np(ops.add_clamp(to_dev(f["a"]), to_dev(f["b"])))
    assert np.array_equal(y.view(np.uint32), f["y"].view(np.uint32))


def test_golden_q8_0(dev):
    from acestep_ops import _lib

    f = _fx("q8_0")
    x = to_dev(f["x"])
    for rounding, key in ((_lib.Q8_0_CPU_X86, "q_x86"), (_lib.Q8_0_REF, "q_ref")):
        dst = DTensor.zeros(f[key].shape, "u8")
        ops.cpy(x, ops.Q8(dst), rounding=rounding)
        assert np.array_equal(to_np(dst), f[key]), key
    rows = to_np(ops.get_rows(ops.Q8(to_dev(f["table"])), to_dev(f["ids"])))
    assert np.array_equal(rows.view(np.uint32), f["rows"].view(np.uint32))


def test_golden_timestep_embedding(dev):
    f = _fx("tsembd")
    t = f["t"]
    y = to_np(ops.timestep_embedding(to_dev(t), 256, 10000))
    tsembd_bar(y, f["y"], t, 256, 10000)
