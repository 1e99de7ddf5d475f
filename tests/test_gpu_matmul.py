"""GPU parity: ggml_mul_mat with Q8_0 weights (mi_q8_0_repack + mi_mul_mat_q8_0)
against the oracle: the matrix-vector kernel (up to 8 rows of x) and the
matrix kernel (more rows: prefill, the DiT).

The oracle is the exact value of ggml-cpu's definition (x quantized with the
x86 Q8_0 quantizer, exact int32 block dots scaled by fp16(d_w) fp16(d_x)),
rounded to float once. The kernel's int32 dots and the d_w * d_x products are
exact in fp32; it rounds once per block (fma into the running sum) and once
per added split, so the bar, written here, is
  |y - ref| <= (K / 32 + 8) * 2^-24 * sum_k |w_k| |x'_k|  (+ 1e-30)
with x' the dequantized quantized x. One quant of x rounded differently moves
y by |d_w d_x q_w|, far above that bound, so the x quantization is checked
bit for bit through y.
"""
import numpy as np
import pytest
from helpers import assert_mul_mat_q8_0, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu


def _check(y, w, x):
    assert_mul_mat_q8_0(y, w, x)


def _run(n, k, m, seed, wscale=1.0, xscale=1.0, wview=None):
    r = np.random.default_rng(seed)
    wf = (r.standard_normal((n, k)) * wscale).astype(np.float32)
    w = orc.quantize_q8_0(wf)
    x = (r.standard_normal((m, k)) * xscale).astype(np.float32)
    if wview is None:
        dw = ops.Q8(to_dev(w))
    else:  # rows of a wider table: row stride wview bytes
        big = np.zeros((n, wview), np.uint8)
        big[:, :w.shape[1]] = w
        dw = ops.Q8(to_dev(big).view(n, wview)[:, :w.shape[1]])
    wr = ops.q8_0_repack(dw)
    y = to_np(ops.mul_mat_q8_0(wr, to_dev(x)))
    _check(y, w, x)
    return w, x, wr


@pytest.mark.parametrize("n,k,m", [(6144, 2560, 8), (2560, 9728, 8), (2560, 4096, 1), (19456, 2560, 4),
                                   (300, 2560, 3), (130, 64, 5), (1, 32, 8), (77, 96, 2)])
def test_decode_shapes(dev, n, k, m):
    """Qwen3-4B decode projections (QKV, down, O, gate/up) at batch 8 / 1 / 4, and
    ragged row counts (a partial last group of 64 rows), one- and two-block rows."""
    print(f"mul_mat q8_0 n={n} k={k} m={m}", flush=True)
    _run(n, k, m, seed=n + k + m)


def test_lm_head_single_split(dev):
    """Many row groups (the LM head's 151669 rows, short rows here): no key split."""
    print("mul_mat q8_0 lm-head rows", flush=True)
    _run(151669, 64, 8, seed=11)


def test_strided_weight_rows_and_scales(dev):
    """Weight rows at a wider stride (a view of a larger table), and inputs with
    large and tiny magnitudes (fp16 scales near their range ends)."""
    print("mul_mat q8_0 strided weights", flush=True)
    _run(200, 256, 6, seed=12, wview=256 // 32 * 34 + 68)
    _run(200, 256, 6, seed=13, wscale=3e3, xscale=1e-3)
    _run(200, 256, 6, seed=14, wscale=1e-4, xscale=50.0)


def test_strided_and_unaligned_x_rows(dev):
    print("mul_mat q8_0 strided x", flush=True)
    r = np.random.default_rng(15)
    n, k, m = 500, 320, 7
    w = orc.quantize_q8_0(r.standard_normal((n, k)).astype(np.float32))
    xbig = r.standard_normal((m, k + 3)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dx = to_dev(xbig)
    y = to_np(ops.mul_mat_q8_0(wr, dx[:, 1:k + 1]))  # rows 4-byte aligned only
    _check(y, w, np.ascontiguousarray(xbig[:, 1:k + 1]))


def test_zero_x_rows_and_repeat_calls_are_identical(dev):
    """A zero row of x gives zeros; the split counters reset, so a second call with
    the same workspace gives bit-identical results."""
    print("mul_mat q8_0 repeat", flush=True)
    r = np.random.default_rng(16)
    n, k, m = 2560, 9728, 8
    w = orc.quantize_q8_0(r.standard_normal((n, k)).astype(np.float32))
    x = r.standard_normal((m, k)).astype(np.float32)
    x[3] = 0.0
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dx = to_dev(x)
    ws = DTensor.empty((ops.mul_mat_q8_0_workspace(wr, dx),), "u8")
    y1 = to_np(ops.mul_mat_q8_0(wr, dx, workspace=ws))
    y2 = to_np(ops.mul_mat_q8_0(wr, dx, workspace=ws))
    assert np.array_equal(y1, y2)
    assert np.all(y1[3] == 0.0)
    _check(y1, w, x)


@pytest.mark.parametrize("n,k,m", [(2048, 2048, 300), (640, 256, 129), (100, 96, 9), (6144, 512, 512),
                                   (70, 32, 1000), (2560, 9728, 520), (2560, 4096, 300)])
def test_matrix_kernel_shapes(dev, n, k, m):
    """More than 8 rows of x (DiT and prefill projections): ragged row tiles of x
    and of the weights, one-block rows, many rows; the narrow Qwen3-4B prefill
    products (n = 2560: O, down), whose few 128 x 128 tiles take key splits added
    by a second launch (2048 x 2048 x 300 takes two)."""
    print(f"mul_mat q8_0 matrix n={n} k={k} m={m}", flush=True)
    _run(n, k, m, seed=n * 7 + k + m)


@pytest.mark.parametrize("m", [8, 300])
def test_subnormal_fp16_scales(dev, m):
    """Weights and x small enough that both block scales are fp16 subnormals
    (|d| < 2^-14; d_x = amax/127 ~ 3e-6, d_w ~ 2e-6), through the matrix-vector
    kernel (8 rows) and the matrix kernel (300 rows), whose scale products come
    from an fp16 MFMA: subnormal inputs must not be flushed."""
    print(f"mul_mat q8_0 subnormal scales m={m}", flush=True)
    w, x, _ = _run(640, 256, m, seed=29 + m, wscale=1e-4, xscale=1e-4)
    dx = np.abs(x.reshape(m, -1, 32)).max(axis=-1) / 127.0
    assert (dx < 2.0 ** -14).all()  # every x scale is an fp16 subnormal
    dw = w.reshape(w.shape[0], -1, 34)[:, :, :2].copy().view(np.float16).astype(np.float32)
    assert (np.abs(dw) < 2.0 ** -14).all()


def test_matrix_kernel_strided_x_and_y(dev):
    print("mul_mat q8_0 matrix strided x/y", flush=True)
    r = np.random.default_rng(17)
    n, k, m = 300, 320, 200
    w = orc.quantize_q8_0(r.standard_normal((n, k)).astype(np.float32))
    xbig = r.standard_normal((m, k + 3)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    ybig = DTensor.zeros((m, n + 5), "f32")
    ops.mul_mat_q8_0(wr, to_dev(xbig)[:, 2:k + 2], out=ybig[:, 1:n + 1])
    yb = to_np(ybig)
    assert np.all(yb[:, 0] == 0) and np.all(yb[:, n + 1:] == 0)
    _check(yb[:, 1:n + 1], w, np.ascontiguousarray(xbig[:, 2:k + 2]))


@pytest.mark.parametrize("n,k,m,swapped", [(2560, 9728, 8, False), (300, 256, 3, True), (640, 256, 129, False),
                                           (100, 96, 1000, True)])
def test_swiglu_prologue_matches_swiglu_then_mul_mat(dev, n, k, m, swapped):
    """mi_mul_mat_q8_0_swiglu (the SwiGLU computed inside the quantization of x)
    against mi_swiglu followed by mi_mul_mat_q8_0: bit-identical, for the decode
    kernel (m <= 8) and the matrix kernel, gate first or second; and the product
    against the oracle on the SwiGLU values the device produced. Gate values down
    to -100 take silu's overflow branch (e^-x = inf, silu = -0)."""
    print(f"mul_mat q8_0 swiglu n={n} k={k} m={m} swapped={swapped}", flush=True)
    r = np.random.default_rng(n + k + m)
    w = orc.quantize_q8_0((r.standard_normal((n, k)) * 0.05).astype(np.float32))
    gu = (r.standard_normal((m, 2 * k)) * 2.0).astype(np.float32)
    gu[:, :: 97] = -100.0
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dgu = to_dev(gu)
    y_f = to_np(ops.mul_mat_q8_0_swiglu(wr, dgu, swapped=swapped))
    ff = ops.swiglu(dgu, swapped=swapped)
    y_u = to_np(ops.mul_mat_q8_0(wr, ff))
    assert np.array_equal(y_f, y_u)
    _check(y_f, w, to_np(ff))


@pytest.mark.parametrize("n,k,m,clamp,inplace", [
    (2560, 9728, 8, False, False),   # Qwen3-4B down projection: key splits summed by the second launch
    (2560, 9728, 8, True, True),     # clamp_fp16, the residual buffer updated in place
    (16448, 256, 4, True, False),    # 257 row groups: splits added in LDS, one launch
    (640, 256, 129, False, False),   # the matrix kernel
    (640, 256, 129, True, True),
    (2560, 9728, 200, True, True),   # the matrix kernel with key splits: the residual added by the split sum
])
def test_swiglu_down_with_residual_add(dev, n, k, m, clamp, inplace):
    """mi_mul_mat_q8_0_swiglu_add against mi_mul_mat_q8_0_swiglu then mi_add /
    mi_add_clamp: bit-identical on every path that forms the product's sum. The
    residual is scaled past the fp16 range in the clamped cases."""
    print(f"mul_mat q8_0 swiglu + add n={n} k={k} m={m} clamp={clamp} inplace={inplace}", flush=True)
    r = np.random.default_rng(n + k + m + int(clamp))
    w = orc.quantize_q8_0((r.standard_normal((n, k)) * 0.05).astype(np.float32))
    gu = (r.standard_normal((m, 2 * k)) * 2.0).astype(np.float32)
    res = (r.standard_normal((m, n)) * (1e5 if clamp else 1.0)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dgu, dres = to_dev(gu), to_dev(res)
    lim = (-65504.0, 65504.0) if clamp else None
    y_f = to_np(ops.mul_mat_q8_0_swiglu_add(wr, dgu, dres, clamp=lim, out=dres if inplace else None))
    mlp = ops.mul_mat_q8_0_swiglu(wr, dgu)
    dres2 = to_dev(res)
    y_u = to_np(ops.add_clamp(dres2, mlp, *lim) if clamp else ops.add(dres2, mlp))
    assert np.array_equal(y_f, y_u)
    if clamp:
        assert (np.abs(res) > 65504.0).any() and np.abs(y_f).max() <= 65504.0


@pytest.mark.parametrize("n,k,m,inplace", [
    (2048, 6144, 8, False),     # decode kernel: splits added in LDS, the gate in the store
    (2048, 6144, 8, True),
    (640, 256, 129, False),     # the matrix kernel
    (2048, 6144, 200, True),    # the matrix kernel with key splits: the gate in the split sum
    (16448, 256, 4, False),     # 257 row groups
])
def test_swiglu_down_with_gated_add(dev, n, k, m, inplace):
    """mi_mul_mat_q8_0_swiglu_gated_add against mi_mul_mat_q8_0_swiglu then
    mi_gated_add: bit-identical on every path that forms the product's sum."""
    print(f"mul_mat q8_0 swiglu + gated add n={n} k={k} m={m} inplace={inplace}", flush=True)
    r = np.random.default_rng(n + k + m + 7)
    w = orc.quantize_q8_0((r.standard_normal((n, k)) * 0.05).astype(np.float32))
    gu = (r.standard_normal((m, 2 * k)) * 2.0).astype(np.float32)
    res = r.standard_normal((m, n)).astype(np.float32)
    gate = (0.7 * r.standard_normal(n)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dgu, dres, dg = to_dev(gu), to_dev(res), to_dev(gate)
    y_f = to_np(ops.mul_mat_q8_0_swiglu_gated_add(wr, dgu, dres, dg, out=dres if inplace else None))
    mlp = ops.mul_mat_q8_0_swiglu(wr, dgu)
    y_u = to_np(ops.gated_add(to_dev(res), mlp, dg))
    assert np.array_equal(y_f, y_u)
    assert np.array_equal(y_u, orc.gated_add(res, to_np(mlp), gate))


def test_swiglu_prologue_strided_rows(dev):
    """gu rows at a stride that is not a multiple of 16 bytes (element loads)."""
    print("mul_mat q8_0 swiglu strided", flush=True)
    r = np.random.default_rng(21)
    n, k, m = 200, 128, 5
    w = orc.quantize_q8_0(r.standard_normal((n, k)).astype(np.float32))
    big = r.standard_normal((m, 2 * k + 1)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dgu = to_dev(big)[:, :2 * k]
    y_f = to_np(ops.mul_mat_q8_0_swiglu(wr, dgu))
    y_u = to_np(ops.mul_mat_q8_0(wr, ops.swiglu(dgu)))
    assert np.array_equal(y_f, y_u)


@pytest.mark.parametrize("n,k,m,view", [(6144, 2560, 8, False), (300, 256, 3, True), (640, 256, 129, False),
                                        (100, 96, 1000, True), (64, 2560, 4100, False), (64, 4096, 4099, True),
                                        (96, 1536, 4096, False)])
def test_rms_norm_prologue_matches_norm_then_mul_mat(dev, n, k, m, view):
    """mi_mul_mat_q8_0_rms_norm (RMSNorm*w computed inside the quantization of x)
    against mi_rms_norm followed by mi_mul_mat_q8_0: bit-identical, for the decode and
    matrix kernels, with a workgroup per row and (4096 rows or more) per 8 rows, a
    ragged last group among them, with 16-byte aligned rows or rows 4 bytes off
    (element loads); rows of very different scales. Then the product against the oracle on the
    normalized rows the device produced."""
    print(f"mul_mat q8_0 rms_norm n={n} k={k} m={m} view={view}", flush=True)
    r = np.random.default_rng(n + k + m + 1)
    w = orc.quantize_q8_0((r.standard_normal((n, k)) * 0.05).astype(np.float32))
    x = r.standard_normal((m, k + (1 if view else 0))).astype(np.float32)
    x *= np.float32(10.0) ** r.integers(-3, 4, (m, 1)).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    dx = to_dev(x)[:, 1:] if view else to_dev(x)
    dnw = to_dev(nw)
    y_f = to_np(ops.mul_mat_q8_0_rms_norm(wr, dx, dnw, 1e-6))
    norm = ops.rms_norm(dx, 1e-6, dnw)
    y_u = to_np(ops.mul_mat_q8_0(wr, norm))
    assert np.array_equal(y_f, y_u)
    _check(y_f, w, to_np(norm))


@pytest.mark.parametrize("n,k,m,add,gated,mod", [
    (4096, 2048, 8, False, False, True),     # decode kernel, norm -> modulate
    (640, 256, 129, False, False, True),     # matrix kernel, a workgroup per row
    (96, 2048, 4100, False, False, True),    # 8 rows per workgroup, ragged last group
    (640, 256, 129, True, True, False),      # gated add -> norm (the cross-attention norm)
    (64, 2048, 4103, True, True, False),
    (640, 256, 129, True, True, True),       # gated add -> norm -> modulate (the FFN norm)
    (64, 2048, 4096, True, True, True),
    (300, 256, 3, True, False, True),        # plain add -> norm -> modulate (after cross attention)
    (64, 256, 4104, True, False, True),
])
def test_adaln_prologue_matches_unfused(dev, n, k, m, add, gated, mod):
    """mi_mul_mat_q8_0_adaln (the DiT's residual add, gated or plain, the RMSNorm*w
    and the AdaLN modulate made inside the quantization of x) against
    mi_add_rms_norm / mi_rms_norm_modulate / mi_rms_norm followed by
    mi_mul_mat_q8_0: the sum and the product bit-identical, for the decode and
    matrix kernels, a workgroup per row and per 8 rows; then the product against
    the oracle on the normalized rows the device produced."""
    print(f"mul_mat q8_0 adaln n={n} k={k} m={m} add={add} gated={gated} mod={mod}", flush=True)
    r = np.random.default_rng(n + k + m + 3)
    w = orc.quantize_q8_0((r.standard_normal((n, k)) * 0.05).astype(np.float32))
    a = r.standard_normal((m, k)).astype(np.float32)
    a *= np.float32(10.0) ** r.integers(-2, 3, (m, 1)).astype(np.float32)
    b = (r.standard_normal((m, k)) * 0.3).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    g = (0.5 * r.standard_normal(k)).astype(np.float32)
    sc = (0.3 * r.standard_normal(k)).astype(np.float32)
    sh = (0.3 * r.standard_normal(k)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    da, db, dnw, dg, dsc, dsh = (to_dev(v) for v in (a, b, nw, g, sc, sh))
    kw = {"gate": dg if gated else None, "scale": dsc if mod else None, "shift": dsh if mod else None}
    if add:
        s_f, y_f = ops.mul_mat_q8_0_adaln(wr, da, dnw, 1e-6, b=db, **kw)
        s_u, n_u = ops.add_rms_norm(da, db, 1e-6, w=dnw, **kw)
        assert np.array_equal(to_np(s_f), to_np(s_u))
    else:
        y_f = ops.mul_mat_q8_0_adaln(wr, da, dnw, 1e-6, scale=dsc, shift=dsh)
        n_u = ops.rms_norm_modulate(da, dnw, dsc, dsh, 1e-6)
    y_u = to_np(ops.mul_mat_q8_0(wr, n_u))
    assert np.array_equal(to_np(y_f), y_u)
    _check(to_np(y_f), w, to_np(n_u))


@pytest.mark.parametrize("n,k,m", [(19456, 2560, 8), (300, 256, 3), (640, 256, 129), (64, 2560, 4103),
                                   (64, 4096, 4096), (64, 256, 4104)])
def test_add_rms_norm_prologue_matches_add_norm_then_mul_mat(dev, n, k, m):
    """mi_mul_mat_q8_0_add_rms_norm (sum = a + b written, RMSNorm*w of it made inside
    the quantization of x) against mi_add_rms_norm followed by mi_mul_mat_q8_0: the
    sum bit-identical, the product bit-identical; then the product against the oracle
    on the normalized rows the device produced."""
    print(f"mul_mat q8_0 add_rms_norm n={n} k={k} m={m}", flush=True)
    r = np.random.default_rng(n + k + m + 2)
    w = orc.quantize_q8_0((r.standard_normal((n, k)) * 0.05).astype(np.float32))
    a = r.standard_normal((m, k)).astype(np.float32)
    b = (r.standard_normal((m, k)) * 0.3).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    wr = ops.q8_0_repack(ops.Q8(to_dev(w)))
    da, db, dnw = to_dev(a), to_dev(b), to_dev(nw)
    s_f, y_f = ops.mul_mat_q8_0_add_rms_norm(wr, da, db, dnw, 1e-6)
    s_u, n_u = ops.add_rms_norm(da, db, 1e-6, w=dnw)
    y_u = to_np(ops.mul_mat_q8_0(wr, n_u))
    assert np.array_equal(to_np(s_f), to_np(s_u))
    assert np.array_equal(to_np(y_f), y_u)
    _check(to_np(y_f), w, to_np(n_u))
