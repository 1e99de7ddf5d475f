"""Writes the golden fixtures in tests/golden/*.npz from the CPU oracle.

The reference's own tests hold no vectors for these ops (ggml is an absent
submodule there), so these fixtures are regression anchors produced by the
oracle, which tests/test_oracle_pinning.py pins independently. Inputs are
seeded, small, and include the edge cases the GPU tests must keep covering:
zero / huge / tiny rows, NaN and +-inf, fp16-range outliers for the clamp,
exact rounding ties for both Q8_0 quantizers, positions up to 8191.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

EPS = 1e-6


def rnd(seed, shape, scale=1.0, mean=0.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale + mean).astype(np.float32)


def norm_rows(seed, rows, n):
    x = rnd(seed, (rows, n))
    x[0] = 0.0                      # all-zero row: scale = 1/sqrt(eps)
    x[1] *= np.float32(1e18)        # squares overflow fp32 range only in double
    x[2] *= np.float32(1e-20)       # squares underflow to 0 in fp32
    x[3, ::7] = np.float32(3e4)
    return x


def rms_norm_modulate_f32():
    x = norm_rows(1, 16, 2048)
    w, sc, sh = rnd(2, (2048,), 0.1, 1.0), rnd(3, (2048,), 0.1), rnd(4, (2048,), 0.1)
    return dict(x=x, w=w, scale=sc, shift=sh, eps=np.float32(EPS),
                y_norm=orc.rms_norm_mul(x, w, EPS), y_mod=orc.rms_norm_modulate(x, w, sc, sh, EPS))


def dit_bf16():
    h = orc.f32_to_bf16(norm_rows(5, 16, 2048)[4:])     # bf16 cannot hold 1e18 squares exactly: skip rows 0-3
    x = orc.f32_to_bf16(rnd(6, (12, 2048)))
    w, sc, sh, g = rnd(7, (2048,), 0.1, 1.0), rnd(8, (2048,), 0.1), rnd(9, (2048,), 0.1), rnd(10, (2048,), 0.1)
    ch = orc.bf16_chain
    ysum = ch(orc.gated_add, h, x, g)
    return dict(h=h, x=x, w=w, scale=sc, shift=sh, gate=g, eps=np.float32(EPS),
                y_mod=ch(orc.rms_norm_modulate, h, w, sc, sh, EPS),
                y_sum=ysum, y_sum_norm=ch(orc.rms_norm_modulate, ysum, w, sc, sh, EPS))


def qk_rope_f32():
    q, k = rnd(11, (4, 32, 128), 2.0), rnd(12, (4, 8, 128), 2.0)
    qw, kw = rnd(13, (128,), 0.1, 1.0), rnd(14, (128,), 0.1, 1.0)
    pos = np.int32([0, 1, 4095, 8191])
    return dict(q=q, k=k, q_w=qw, k_w=kw, pos=pos, theta=np.float32(1e6), eps=np.float32(EPS),
                q_out=orc.qk_norm_rope(q, qw, pos, EPS, 128, 1e6), k_out=orc.qk_norm_rope(k, kw, pos, EPS, 128, 1e6))


def qk_rope_bf16():
    q, k = orc.f32_to_bf16(rnd(15, (6, 16, 128))), orc.f32_to_bf16(rnd(16, (6, 8, 128)))
    qw, kw = rnd(17, (128,), 0.1, 1.0), rnd(18, (128,), 0.1, 1.0)
    pos = np.int32([0, 7, 1000, 2999, 3000, 5999])
    f = orc.bf16_chain
    return dict(q=q, k=k, q_w=qw, k_w=kw, pos=pos, theta=np.float32(1e4), eps=np.float32(EPS),
                q_out=f(orc.qk_norm_rope, q, qw, pos, EPS, 128, 1e4),
                k_out=f(orc.qk_norm_rope, k, kw, pos, EPS, 128, 1e4))


def swiglu_f32():
    gu = rnd(19, (8, 2 * 768), 4.0)
    gu[0, :9] = np.float32([0.0, -0.0, 100.0, -100.0, -90.0, 88.0, np.inf, -np.inf, np.nan])
    gu[1, :4] = np.float32([3.4e38, -3.4e38, 1e-30, -1e-30])
    return dict(gu=gu, y=orc.swiglu(gu), y_swapped=orc.swiglu(gu, swapped=True))


def add_clamp_f32():
    a, b = rnd(20, (16, 1024)), rnd(21, (16, 1024))
    r = np.random.default_rng(22)
    idx = r.choice(a.size, 64, replace=False)
    a.reshape(-1)[idx] = (r.standard_normal(64) * 1e5).astype(np.float32)
    a[0, :4] = np.float32([np.nan, np.inf, -np.inf, 65504.0])
    b[0, 3] = np.float32(1.0)
    return dict(a=a, b=b, y=orc.add_clamp(a, b))


def q8_0():
    blocks = [np.arange(32, dtype=np.float32) - 16.0]
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:] = np.arange(1, 32, dtype=np.float32) + 0.5          # exact .5 ties (id = 1 in both variants)
    blocks += [t, -t, np.zeros(32, np.float32), rnd(23, (32,), 1e-6), rnd(24, (32,), 1e-10), rnd(25, (32,), 6e4)]
    blocks += list(rnd(26, (25, 32)))
    x = np.stack(blocks).reshape(4, 256)
    table = orc.quantize_q8_0(rnd(27, (64, 256), 0.02), "ref")
    ids = np.int32([0, 63, 5, 5, 17, 40])
    return dict(x=x, q_x86=orc.quantize_q8_0(x, "x86"), q_ref=orc.quantize_q8_0(x, "ref"), table=table, ids=ids,
                rows=orc.get_rows(table, orc.Q8_0, 256, ids))


def tsembd():
    t = np.float32([0.0, 0.001, 0.5, 1.0, 250.0, 999.0])
    return dict(t=t, y=orc.timestep_embedding(t, 256, 10000))


FIXTURES = {
    "rms_norm_modulate_f32": rms_norm_modulate_f32,
    "dit_bf16": dit_bf16,
    "qk_rope_f32": qk_rope_f32,
    "qk_rope_bf16": qk_rope_bf16,
    "swiglu_f32": swiglu_f32,
    "add_clamp_f32": add_clamp_f32,
    "q8_0": q8_0,
    "tsembd": tsembd,
}


def main():
    orc.set_threads(1)
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} B)")


if __name__ == "__main__":
    main()
