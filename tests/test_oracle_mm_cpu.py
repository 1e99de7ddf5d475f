"""Pinning the Q8_0 matrix-product oracle (orc_mul_mat_q8_0) without ggml.

Each check is fixed by something other than the oracle's own formula:
  - the float64 product of the dequantized matrices, a different association
    of the same sum (per element instead of per block integer dots);
  - a closed form for a unit weight block;
  - the quantizer of x is the x86 one, separated from the reference
    quantizer by tie blocks;
  - additivity over concatenated K ranges;
  - zero rows of x give zero.
Planting each of these mistakes in a copy of the oracle fails at least one
test: the reference quantizer for x, a dropped d_x, d_w of block 0 for every
block, quants read as unsigned, the output transposed, blocks of row 0 for
every weight row.
"""
import numpy as np
from oracle import oracle as orc


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _bound(wf, xf):
    """|w| |x| sums: an upper bound of sum_b |d_w d_x isum_b| per output"""
    return np.abs(xf).astype(np.float64) @ np.abs(wf).astype(np.float64).T


def test_equals_float64_product_of_dequantized():
    n, k, m = 37, 320, 5
    w = orc.quantize_q8_0(_rand((n, k), 1))
    x = _rand((m, k), 2, 3.0)
    y = orc.mul_mat_q8_0(w, x)
    wf = orc.dequantize_q8_0(w).astype(np.float64)
    xf = orc.dequantize_q8_0(orc.quantize_q8_0(x, "x86")).astype(np.float64)
    ref = xf @ wf.T
    assert y.shape == (m, n)
    assert np.all(np.abs(y - ref) <= 2.0 ** -24 * np.abs(ref) + 1e-12 * _bound(wf, xf))


def test_unit_weight_block_closed_form():
    k = 64
    w = np.zeros((3, k // 32 * 34), np.uint8)
    one = np.array([0x3C00], np.uint16).view(np.uint8)  # fp16 1.0
    for j, (blk, i) in enumerate([(0, 0), (1, 5), (1, 31)]):
        w[j, blk * 34:blk * 34 + 2] = one
        w[j, blk * 34 + 2 + i] = 1  # q_w = e_i in block blk
    x = _rand((2, k), 3)
    xq = orc.quantize_q8_0(x, "x86")
    y = orc.mul_mat_q8_0(w, x)
    for r in range(2):
        for j, (blk, i) in enumerate([(0, 0), (1, 5), (1, 31)]):
            d_x = orc.f16_to_f32(xq[r, blk * 34:blk * 34 + 2].view(np.uint16))[0]
            q_x = xq[r, blk * 34 + 2 + i].astype(np.int8)
            assert y[r, j] == np.float32(np.float64(d_x) * int(q_x))


def test_x_is_quantized_with_the_x86_rounding():
    """Blocks whose scaled values hit exact .5 ties: the x86 from_float rounds
    them to even, quantize_row_q8_0_ref away from zero."""
    blk = np.zeros(32, np.float32)
    blk[0] = 127.0
    blk[1:] = (np.arange(1, 32) % 9).astype(np.float32) + 0.5
    x = np.tile(blk, 4).reshape(1, 128)
    w = orc.quantize_q8_0(_rand((16, 128), 4))
    x86 = orc.dequantize_q8_0(orc.quantize_q8_0(x, "x86"))
    ref = orc.dequantize_q8_0(orc.quantize_q8_0(x, "ref"))
    assert not np.array_equal(x86, ref)
    wf = orc.dequantize_q8_0(w).astype(np.float64)
    y = orc.mul_mat_q8_0(w, x)
    assert np.allclose(y, (x86.astype(np.float64) @ wf.T), rtol=1e-6, atol=1e-6)
    assert not np.allclose(y, (ref.astype(np.float64) @ wf.T), rtol=1e-6, atol=1e-6)


def test_additive_over_k_ranges():
    n, m = 9, 3
    w1, w2 = orc.quantize_q8_0(_rand((n, 96), 5)), orc.quantize_q8_0(_rand((n, 64), 6))
    x1, x2 = _rand((m, 96), 7), _rand((m, 64), 8)
    y = orc.mul_mat_q8_0(np.concatenate([w1, w2], axis=1), np.concatenate([x1, x2], axis=1))
    y12 = orc.mul_mat_q8_0(w1, x1).astype(np.float64) + orc.mul_mat_q8_0(w2, x2).astype(np.float64)
    assert np.allclose(y, y12, rtol=1e-6, atol=1e-6)


def test_zero_rows_of_x_give_zero():
    w = orc.quantize_q8_0(_rand((11, 64), 9))
    x = _rand((3, 64), 10)
    x[1] = 0.0
    y = orc.mul_mat_q8_0(w, x)
    assert np.all(y[1] == 0.0) and np.any(y[0] != 0.0)
