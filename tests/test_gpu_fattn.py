"""GPU parity: ggml_flash_attn_ext (mi_flash_attn_ext) against the oracle.

The oracle is the exact value of ggml-cpu's definition in double: q converted
to K's dot type (fp16 / bf16 / Q8_0 x86), s = scale * q.k + mask with -inf keys
skipped, softmax, p.V. The kernels compute in fp32; the bar is the error bound
derived from their arithmetic, element by element (tests/fa_bound.py: the dot
products' and exp's roundings as relative errors of each key's weight, the
16-bit P parts of the matrix-core path, the accumulation of o and l, the final
division). Rows whose keys are all masked must be NaN, as ggml's 0 * (1/0)
makes them.

For an F16 V, ggml-cpu itself accumulates the output in fp16 one key at a
time; that variant of the oracle (flash_attn_ext_f16acc) carries its own
rounding errors, and the kernel's result must lie within the sum of the two
bounds of it as well.
"""
import numpy as np
import pytest
from fa_bound import fa_bound
from helpers import to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu


def _rng(seed):
    return np.random.default_rng(seed)


def _kv(x, kt):
    """host float array (..., D) -> (device operand, float values the oracle sees)"""
    if kt == "q8_0":
        qb = orc.quantize_q8_0(x, "x86")
        return ops.Q8(to_dev(qb)), orc.dequantize_q8_0(qb)
    if kt == "f16":
        h = orc.f32_to_f16(x)
        return to_dev(h, f16=True), orc.f16_to_f32(h)
    if kt == "bf16":
        h = orc.f32_to_bf16(x)
        return to_dev(h, bf16=True), orc.bf16_to_f32(h)
    return to_dev(x), x


def _q(x, qt):
    if qt == "bf16":
        h = orc.f32_to_bf16(x)
        return to_dev(h, bf16=True), orc.bf16_to_f32(h)
    return to_dev(x), x


def _mask_dev(m):
    """float mask (values exactly representable in fp16) -> device F16, oracle floats"""
    h = orc.f32_to_f16(m)
    return to_dev(h, f16=True), orc.f16_to_f32(h)


def _check(y, ref, bound):
    """y, ref, bound (N, n_q, Nh, D): NaN rows where the oracle has them, else
    |y - ref| <= bound element by element."""
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(y), nan_ref), "NaN rows differ"
    assert np.array_equal(np.isnan(bound), nan_ref), "bound and oracle disagree on fully masked rows"
    err = np.abs(y.astype(np.float64) - ref)[~nan_ref]
    b = bound[~nan_ref]
    if err.size:
        worst = int(np.argmax(err / b))
        print(f"  max |y - ref| {err.max():.3e}; largest error / bound {err[worst] / b[worst]:.3f}", flush=True)
        assert np.all(err <= b), f"{int((err > b).sum())} elements beyond the bound (worst {err[worst]:.3e} > {b[worst]:.3e})"


def _uses_mfma(kt, D, n_q, Nh, Nkv, n_kv, mask=None):
    """The launch plan's choice of a matrix-core kernel (flash_attn_plan), as
    fa_bound's mfma argument: F16/BF16/Q8_0 K/V at D = 128 with 64 or more query
    rows per KV head ("prefill"; Q8_0 rows 4-byte aligned, as every cache here
    has), or one query position, at most 16 heads per KV head and a mask row
    shared by every head ("dec"; Q8_0 rows 8-byte aligned). They keep P (or P
    times V's block scale) as 16-bit parts."""
    if kt not in ("f16", "bf16", "q8_0") or D != 128 or n_kv <= 0:
        return False
    if n_q == 1 and Nh // Nkv <= 16 and (mask is None or mask.shape[1] == 1):
        return "dec"
    return "prefill" if n_q * (Nh // Nkv) >= 64 else False


def _run(N, Nh, Nkv, n_q, n_kv, D, kt, qt="f32", mask=None, scale=None, seed=0, Nk3=None, kview=None):
    Nk3 = Nk3 or N
    r = _rng(seed)
    q = r.standard_normal((N, Nh, n_q, D)).astype(np.float32)
    k = r.standard_normal((Nk3, Nkv, n_kv, D)).astype(np.float32)
    v = r.standard_normal((Nk3, Nkv, n_kv, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    dq, qf = _q(q, qt)
    if kview is None:
        dk, kf = _kv(k, kt)
        dv, vf = _kv(v, kt)
    else:  # views of the first n_kv slots of larger caches
        pad = np.zeros((Nk3, Nkv, kview - n_kv, D), np.float32)
        dk_full, kf_full = _kv(np.concatenate([k, pad + 7.0], axis=2), kt)
        dv_full, vf_full = _kv(np.concatenate([v, pad - 7.0], axis=2), kt)
        sl = (slice(None), slice(None), slice(0, n_kv))
        dk = ops.Q8(dk_full.data[sl]) if kt == "q8_0" else dk_full[sl]
        dv = ops.Q8(dv_full.data[sl]) if kt == "q8_0" else dv_full[sl]
        kf, vf = kf_full[:, :, :n_kv], vf_full[:, :, :n_kv]
    dm, mf = (None, None) if mask is None else _mask_dev(mask)
    y = to_np(ops.flash_attn_ext(dq, dk, dv, dm, float(scale)))
    rep = N // Nk3  # the oracle takes one KV batch per q batch (ggml: KV batch b // rep)
    ref = orc.flash_attn_ext(qf, np.repeat(kf, rep, axis=0), np.repeat(vf, rep, axis=0), mf, float(scale), kt)
    bound = fa_bound(qf, kf, vf, mf, float(scale), kt, _uses_mfma(kt, D, n_q, Nh, Nkv, n_kv, mf))
    _check(y, ref, bound)
    if kt == "f16":  # ggml-cpu's own F16-V result: within its carried fp16 errors plus our bound
        y16, bud = orc.flash_attn_ext_f16acc(qf, np.repeat(kf, rep, axis=0),
                                             np.repeat(orc.f32_to_f16(vf), rep, axis=0), mf, float(scale), kt)
        fin = ~np.isnan(ref)
        assert np.array_equal(np.isnan(y16), ~fin)
        slack = 1e-5 * float(np.abs(vf).max())  # its fp32 softmax arithmetic
        assert np.all(np.abs(y - y16)[fin] <= (bound + bud)[fin] + slack)
    return y, ref


def _decode_mask(N, n_kv, lens):
    m = np.zeros((N, 1, 1, n_kv), np.float32)
    for b, L in enumerate(lens):
        m[b, 0, 0, L:] = -np.inf
    return m


@pytest.mark.parametrize("kt", ["q8_0", "f16", "bf16", "f32"])
def test_decode_poisoned_slots_past_each_length(dev, kt):
    """Decode over caches whose slots past each sequence's length hold NaN bytes
    (stale or unwritten cache rows), inside tiles that also hold live keys and in
    whole dead tiles: ggml never reads masked keys, so the output stays finite."""
    N, Nh, Nkv, n_kv, D = 3, 32, 8, 1024, 128
    print(f"fa decode poisoned slots kt={kt}", flush=True)
    lens = [1, 513, 1000]
    r = _rng(21)
    q = r.standard_normal((N, Nh, 1, D)).astype(np.float32)
    k = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    v = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    for b, L in enumerate(lens):
        k[b, :, L:] = np.nan
        v[b, :, L:] = np.nan
    dk, kf = _kv(k, kt)
    dv, vf = _kv(v, kt)
    dm, mf = _mask_dev(_decode_mask(N, n_kv, lens))
    y = to_np(ops.flash_attn_ext(to_dev(q), dk, dv, dm, 0.125))
    ref = orc.flash_attn_ext(q, kf, vf, mf, 0.125, kt)
    assert np.isfinite(y).all() and np.isfinite(ref).all()
    _check(y, ref, fa_bound(q, np.nan_to_num(kf), np.nan_to_num(vf), mf, 0.125, kt,
                            _uses_mfma(kt, D, 1, Nh, Nkv, n_kv, mf)))


@pytest.mark.parametrize("kt", ["q8_0", "f16", "bf16", "f32"])
@pytest.mark.parametrize("qt", ["f32", "bf16"])
def test_decode_gqa_per_sequence_lengths(dev, kt, qt):
    """Qwen3-4B decode shape (32/8 heads x 128), 4 sequences of different lengths over a
    1280-slot read (the 256-bucketed length), cache views of a 2048-slot cache."""
    N, n_kv = 4, 1280
    print(f"fa decode kt={kt} qt={qt}", flush=True)
    lens = [1, 300, 1025, 1280]
    _run(N, 32, 8, 1, n_kv, 128, kt, qt, mask=_decode_mask(N, n_kv, lens), seed=1, kview=2048)


@pytest.mark.parametrize("rk,masked,kt,qt", [(16, False, "f16", "f32"), (1, True, "bf16", "bf16"),
                                               (2, False, "bf16", "f32"), (8, True, "f16", "bf16")])
def test_decode_heads_per_kv_head(dev, rk, masked, kt, qt):
    """One query position with 1 to 16 query heads per KV head (the decode
    kernel pads them to 16), with and without a mask, over a ragged 777 keys."""
    print(f"fa decode rk={rk} masked={masked} kt={kt} qt={qt}", flush=True)
    N, Nkv, n_kv = 3, 2, 777
    mask = _decode_mask(N, n_kv, [777, 40, 500]) if masked else None
    _run(N, Nkv * rk, Nkv, 1, n_kv, 128, kt, qt, mask=mask, seed=31 + rk)


@pytest.mark.parametrize("kt,qt,rk,n_kv", [("f16", "f32", 4, 20), ("bf16", "bf16", 16, 32), ("f16", "bf16", 1, 7)])
def test_decode_single_split_and_fully_masked_sequence(dev, kt, qt, rk, n_kv):
    """The matrix-core decode kernel over at most 32 keys: one key split, so
    the kernel writes the output itself (no partials, no merge launch). The
    last sequence has every key masked: its rows are NaN (1/0 row sum)."""
    print(f"fa decode one split kt={kt} qt={qt} rk={rk} n_kv={n_kv}", flush=True)
    N, Nkv = 3, 2
    assert _uses_mfma(kt, 128, 1, Nkv * rk, Nkv, n_kv, _decode_mask(N, n_kv, [n_kv, 3, 0]))
    y, _ = _run(N, Nkv * rk, Nkv, 1, n_kv, 128, kt, qt, mask=_decode_mask(N, n_kv, [n_kv, 3, 0]), seed=41 + rk)
    assert np.isnan(y[2]).all() and np.isfinite(y[:2]).all()


@pytest.mark.parametrize("kt,n_kv", [("f16", 24), ("bf16", 700)])
def test_decode_kv_and_mask_batch_broadcast(dev, kt, n_kv):
    """Decode with K/V shared by pairs of query batches (batch b reads KV batch
    b / 2) and a mask of 2 batches broadcast over 4 (batch b reads mask b % 2),
    with one and with several key splits."""
    print(f"fa decode broadcasts kt={kt} n_kv={n_kv}", flush=True)
    m = _decode_mask(2, n_kv, [n_kv, n_kv // 3])
    _run(4, 8, 2, 1, n_kv, 128, kt, "f32", mask=m, seed=51, Nk3=2)


@pytest.mark.parametrize("layout", ["contiguous", "slot_major"])
def test_decode_q8_row_layouts_ragged(dev, layout):
    """Q8_0 decode over 777 keys (the last 32-key tile holds 9: an odd number of
    136-byte rows) in two cache layouts: each KV head's rows contiguous, and the
    KV heads of a slot side by side (K/V views with a 1088-byte key stride)."""
    print(f"fa decode q8_0 layout={layout}", flush=True)
    N, Nh, Nkv, n_kv, D = 3, 32, 8, 777, 128
    r = _rng(61)
    q = r.standard_normal((N, Nh, 1, D)).astype(np.float32)
    k = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    v = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    if layout == "contiguous":
        dk, kf = _kv(k, "q8_0")
        dv, vf = _kv(v, "q8_0")
    else:
        kq = orc.quantize_q8_0(np.ascontiguousarray(k.transpose(0, 2, 1, 3)), "x86")  # (N, n_kv, Nkv, 136)
        vq = orc.quantize_q8_0(np.ascontiguousarray(v.transpose(0, 2, 1, 3)), "x86")
        dk = ops.Q8(to_dev(kq).permute(0, 2, 1, 3))
        dv = ops.Q8(to_dev(vq).permute(0, 2, 1, 3))
        assert dk.data.strides[2] == Nkv * 136
        kf = orc.dequantize_q8_0(kq).transpose(0, 2, 1, 3)
        vf = orc.dequantize_q8_0(vq).transpose(0, 2, 1, 3)
    m = _decode_mask(N, n_kv, [777, 9, 300])
    dm, mf = _mask_dev(m)
    y = to_np(ops.flash_attn_ext(to_dev(q), dk, dv, dm, 0.125))
    ref = orc.flash_attn_ext(q, kf, vf, mf, 0.125, "q8_0")
    _check(y, ref, fa_bound(q, kf, vf, mf, 0.125, "q8_0", _uses_mfma("q8_0", D, 1, Nh, Nkv, n_kv, mf)))


@pytest.mark.parametrize("kt", ["q8_0", "f16"])
def test_decode_long_kv_splits(dev, kt):
    """8192 keys: the key range is split over many waves and merged."""
    print(f"fa long kv kt={kt}", flush=True)
    N, n_kv = 2, 8192
    _run(N, 8, 2, 1, n_kv, 128, kt, "bf16", mask=_decode_mask(N, n_kv, [8192, 5000]), seed=2)


@pytest.mark.parametrize("D,kt", [(64, "f16"), (64, "q8_0"), (64, "f32"), (128, "bf16"), (256, "f16"),
                                  (256, "q8_0")])
def test_prefill_window_mask_ragged(dev, D, kt):
    """DiT-style self attention: 37 queries x 300 keys (ragged tiles), a sliding-window +
    padding mask, 16/8 heads, 2 batch elements sharing the mask."""
    print(f"fa prefill D={D} kt={kt}", flush=True)
    n_q, n_kv, win, real = 37, 300, 64, 290
    m = np.zeros((1, 1, 40, n_kv), np.float32)  # padded to 40 query rows, as ggml pads the mask
    for i in range(n_q):
        for j in range(n_kv):
            if abs(i * 8 - j) > win or j >= real:
                m[0, 0, i, j] = -np.inf
    _run(2, 16, 8, n_q, n_kv, D, kt, "f32", mask=m, seed=3)


def test_finite_mask_values_per_head(dev):
    """A mask with finite biases, one per (head, query): mne2 = Nh, mne3 = 1."""
    print("fa finite per-head mask", flush=True)
    r = _rng(4)
    m = np.round(r.uniform(-3, 3, (1, 4, 5, 200)) * 64) / 64  # exact in fp16
    _run(3, 4, 2, 5, 200, 128, "f16", mask=m.astype(np.float32), seed=4)


def test_no_mask_and_kv_batch_broadcast(dev):
    """No mask; K/V shared by pairs of batch elements (ne3 broadcast, rk3 = 2)."""
    print("fa no mask, rk3 = 2", flush=True)
    _run(4, 8, 8, 3, 100, 128, "q8_0", "f32", mask=None, seed=5, Nk3=2)


def test_mfma_prefill_q8_poisoned_slots_past_each_length(dev):
    """Prefill over a Q8_0 cache whose slots past each sequence's length hold NaN
    scales (unwritten cache rows), inside a tile that also holds live keys and in
    whole dead tiles: the matrix-core kernel reads a non-finite V scale as 0, so
    keys masked for a row (p = 0) leave the output finite, as ggml never reads them."""
    print("fa mfma prefill q8_0 poisoned slots", flush=True)
    N, Nh, Nkv, n_q, n_kv, D = 2, 8, 2, 40, 200, 128
    lens = [200, 90]
    assert _uses_mfma("q8_0", D, n_q, Nh, Nkv, n_kv) == "prefill"
    r = _rng(23)
    q = r.standard_normal((N, Nh, n_q, D)).astype(np.float32)
    k = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    v = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    m = np.full((N, 1, n_q, n_kv), -np.inf, np.float32)
    for b, L in enumerate(lens):
        k[b, :, L:] = np.nan
        v[b, :, L:] = np.nan
        for i in range(n_q):
            m[b, 0, i, :L - n_q + i + 1] = 0.0   # causal: the new tokens are the last n_q of the sequence
    dk, kf = _kv(k, "q8_0")
    dv, vf = _kv(v, "q8_0")
    assert np.isnan(kf[1, :, 90:]).all() and np.isnan(vf[1, :, 90:]).all()
    dm, mf = _mask_dev(m)
    y = to_np(ops.flash_attn_ext(to_dev(q), dk, dv, dm, 0.125))
    ref = orc.flash_attn_ext(q, kf, vf, mf, 0.125, "q8_0")
    assert np.isfinite(y).all() and np.isfinite(ref).all()
    _check(y, ref, fa_bound(q, np.nan_to_num(kf), np.nan_to_num(vf), mf, 0.125, "q8_0", "prefill"))


@pytest.mark.parametrize("kt", ["q8_0", "f16"])
def test_mfma_kv_batch_broadcast_and_cache_view(dev, kt):
    """The matrix-core path with K/V shared by pairs of batch elements (rk3 = 2, GQA 4:1,
    160 rows per KV head), and over views of the first 150 slots of 200-slot caches whose
    other slots hold different values."""
    print(f"fa mfma rk3 = 2 / cache view kt={kt}", flush=True)
    assert _uses_mfma(kt, 128, 40, 8, 2, 150) == "prefill"
    _run(4, 8, 2, 40, 150, 128, kt, "f32", mask=None, seed=12, Nk3=2)
    _run(2, 8, 2, 40, 150, 128, kt, "bf16", mask=None, seed=13, kview=200)


def test_fully_masked_rows_and_poisoned_masked_keys(dev):
    """Rows with every key masked are NaN; keys masked for every row are never read, so
    NaN bytes there do not reach the output."""
    print("fa fully masked rows / poisoned keys", flush=True)
    N, Nh, Nkv, n_q, n_kv, D = 2, 4, 4, 2, 96, 128
    r = _rng(6)
    q = r.standard_normal((N, Nh, n_q, D)).astype(np.float32)
    k = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    v = r.standard_normal((N, Nkv, n_kv, D)).astype(np.float32)
    m = np.zeros((N, 1, n_q, n_kv), np.float32)
    m[0, 0, 1, :] = -np.inf               # b=0, query 1: all keys masked
    m[1, 0, :, 40:70] = -np.inf           # b=1: keys 40..69 masked for both queries
    kh, vh = orc.f32_to_f16(k), orc.f32_to_f16(v)
    kh[1, :, 40:70] = 0x7E00              # NaN bytes in the masked keys
    vh[1, :, 40:70] = 0x7E00
    dm, mf = _mask_dev(m)
    y = to_np(ops.flash_attn_ext(to_dev(q), to_dev(kh, f16=True), to_dev(vh, f16=True), dm, 0.125))
    kf, vf = orc.f16_to_f32(kh), orc.f16_to_f32(vh)
    ref = orc.flash_attn_ext(q, kf, vf, mf, 0.125, "f16")
    assert np.isnan(y[0, 1]).all() and np.isnan(ref[0, 1]).all()
    assert np.isfinite(y[1]).all()
    _check(y, ref, fa_bound(q, np.nan_to_num(kf), np.nan_to_num(vf), mf, 0.125, "f16",
                            _uses_mfma("f16", D, n_q, Nh, Nkv, n_kv, mf)))


def test_empty_key_range_is_nan(dev):
    print("fa n_kv = 0", flush=True)
    q = DTensor.from_numpy(np.ones((1, 2, 1, 64), np.float32))
    k = DTensor.empty((1, 2, 0, 64), "f16")
    y = to_np(ops.flash_attn_ext(q, k, k, None, 1.0))
    assert np.isnan(y).all()


@pytest.mark.parametrize("kt,qt,rk,masked", [("bf16", "bf16", 2, False), ("bf16", "f32", 2, "window"),
                                              ("f16", "f32", 4, "window"), ("f16", "bf16", 2, False),
                                              ("bf16", "bf16", 2, "zero"), ("f16", "f32", 4, "one_key"),
                                              ("q8_0", "f32", 4, "window"), ("q8_0", "bf16", 2, False),
                                              ("q8_0", "f32", 2, "zero"), ("q8_0", "f32", 4, "one_key")])
def test_mfma_prefill(dev, kt, qt, rk, masked):
    """The matrix-core path (128 query rows per workgroup, 64-key tiles): 203 query
    positions x rk heads per KV head (a ragged last row block), 333 keys (a ragged last
    tile), 2 batch elements, with no mask, a window mask, an all-zero mask (every
    workgroup takes the loop without mask reads), or a zero mask with one -inf key in
    one query position (its workgroup reads the mask, the others do not). Q8_0 K/V take
    the kernel's int8 score and split-V form."""
    print(f"fa mfma prefill kt={kt} qt={qt} rk={rk} masked={masked}", flush=True)
    n_q, n_kv, nkv = 203, 333, 2
    mask = None
    if masked == "window":
        i = np.arange(n_q)[:, None]
        j = np.arange(n_kv)[None, :]
        mask = np.where(np.abs(i * 1.6 - j) <= 70, 0.0, -np.inf).astype(np.float32)[None, None]
        mask[..., 5, :] = -np.inf  # one query position with every key masked: NaN rows
    elif masked == "zero":
        mask = np.zeros((1, 1, n_q, n_kv), np.float32)
    elif masked == "one_key":
        mask = np.zeros((1, 1, n_q, n_kv), np.float32)
        mask[..., 150, 77] = -np.inf
    _run(2, nkv * rk, nkv, n_q, n_kv, 128, kt, qt, mask=mask, seed=7)


@pytest.mark.parametrize("kt,n_kv,masked", [("bf16", 333, True), ("f16", 269, False), ("q8_0", 269, True)])
def test_mfma_tail_split(dev, kt, n_kv, masked):
    """More 128-row work items than two rounds of resident workgroups fill, with a last
    round at most half full: those last items run as two halves of the key tiles and a
    second kernel merges the halves. 16 items over a full round (2 x 8 KV heads x one
    extra row block, the last one ragged), an even and an odd number of key tiles; the
    masked case has rows whose second half has no live key, and a fully masked row."""
    # the smallest such shape on this device: the workspace holds the partials of the
    # split items after the mask summary, so it grows past the summary exactly then
    qall = DTensor.empty((2, 16, 64 * 400, 128), "f32")
    kv = ops.Q8(DTensor.empty((2, 8, n_kv, 136), "u8")) if kt == "q8_0" else DTensor.empty((2, 8, n_kv, 128), kt)
    n_q = None
    for rblk in range(2, 400):
        nq = 64 * rblk - 28  # rows = 2 n_q = 128 rblk - 56: a ragged last row block
        msum = -(-(2 * 16 * ((nq + 15) // 16) * ((n_kv + 63) // 64)) // 256) * 256
        ws = ops.flash_attn_workspace(qall[:, :, :nq], kv, kv)
        if ws > msum:
            assert ws == msum + (ws - msum) // (2 * 128 * 132 * 4) * (2 * 128 * 132 * 4)
            n_q = nq
            break
    assert n_q is not None
    print(f"fa mfma tail split kt={kt} n_q={n_q} n_kv={n_kv} masked={masked}", flush=True)
    mask = None
    if masked:
        i = np.arange(n_q)[:, None]
        j = np.arange(n_kv)[None, :]
        mask = np.where(np.abs(i * (n_kv / n_q) - j) <= 40, 0.0, -np.inf).astype(np.float32)[None, None]
        mask[..., 7, :] = -np.inf
    _run(2, 16, 8, n_q, n_kv, 128, kt, "bf16", mask=mask, seed=11)


def _dit_window_mask(S, win, real):
    """The DiT self-attention mask of a sliding-window layer (dit-sampler.h:253-274):
    0 where both positions are real (< real) and |qi - ki| <= win, else -inf;
    [ki, qi] per batch element."""
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    ok = (i < real) & (j < real) & ((win <= 0) | (S <= win) | (np.abs(i - j) <= win))
    return np.where(ok, 0.0, -np.inf).astype(np.float32)


@pytest.mark.parametrize("S,win,real", [(3000, 128, 2950), (3000, 0, 3000)])
def test_dit_self_attention_full_size(dev, S, win, real):
    """The DiT's self attention as the reference runs it (dit-graph.h:201-231):
    S = T / 2 = 3000 tokens per element of the CFG pair (T = 6000 frames at
    patch size 2), 16/8 heads x 128, F32 q as a permuted view of the rope
    output [D, Nh, S, N] -> [D, S, Nh, N], K/V cast to F16, and the F16 mask of
    a sliding-window layer (window 128, the last 50 positions padding: their
    query rows have every key masked and are NaN) or of a full-attention layer
    without padding (all zero). The whole problem runs on the device; 40 query
    positions (window edges, padding edges, both ends) x both CFG elements x
    all 16 heads are checked against the oracle under the kernel's bound."""
    print(f"fa dit self attention S={S} win={win} real={real}", flush=True)
    N, Nh, Nkv, D = 2, 16, 8, 128
    r = _rng(61)
    q = r.standard_normal((N, S, Nh, D), dtype=np.float32)      # rope output rows [D, Nh, S, N]
    k = r.standard_normal((N, Nkv, S, D), dtype=np.float32)
    v = r.standard_normal((N, Nkv, S, D), dtype=np.float32)
    m = np.broadcast_to(_dit_window_mask(S, win, real), (N, 1, S, S))
    dq = to_dev(q).permute(0, 2, 1, 3)                            # (N, Nh, S, D) view
    dk, kf = _kv(k, "f16")
    dv, vf = _kv(v, "f16")
    dm, mf = _mask_dev(np.ascontiguousarray(m))
    scale = 1.0 / np.sqrt(D)
    y = to_np(ops.flash_attn_ext(dq, dk, dv, dm, float(scale)))   # (N, S, Nh, D)
    qs = np.unique(np.r_[0, 1, 63, 64, 127, 128, 129, 255, 256, 1000, 1499, 1500, 2047, 2048,
                         real - 130, real - 129, real - 128, real - 2, real - 1, real, real + 1, S - 2, S - 1,
                         r.integers(0, S, 17)])
    qs = qs[(qs >= 0) & (qs < S)]
    qf = np.ascontiguousarray(q[:, qs].transpose(0, 2, 1, 3))     # (N, Nh, len(qs), D)
    ms = np.ascontiguousarray(mf[:, :, qs])
    ref = orc.flash_attn_ext(qf, kf, vf, ms, float(scale), "f16")
    bound = fa_bound(qf, kf, vf, ms, float(scale), "f16", mfma=True)
    assert _uses_mfma("f16", D, S, Nh, Nkv, S, mf)
    _check(y[:, qs], ref, bound)
    if real < S:
        assert np.isnan(y[:, real:]).all() and np.isfinite(y[:, :real]).all()


@pytest.mark.parametrize("kt", ["q8_0", "f16"])
def test_lm_prefill_attention_full_size(dev, kt):
    """The LM's prefill attention over its KV cache at the Qwen3-4B batched-prefill
    size (qwen3-lm.h:414-417; songgen-lelm-gen.h:276-277): 2 sequences x 2048 new
    tokens from slot 0, 32/8 heads x 128, F32 q as the permuted rope output, K/V
    as views of the first 2048 slots of 4096-slot caches (Q8_0 or F16), the
    causal F16 mask. The whole call runs on the device (4096 work items of the
    matrix-core kernel, longest first); 36 query positions (both ends, tile and
    row-block edges) x both sequences x all 32 heads are checked against the
    oracle under the kernel's bound."""
    print(f"fa lm prefill full size kt={kt}", flush=True)
    N, Nh, Nkv, D, S, SLOTS = 2, 32, 8, 128, 2048, 4096
    r = _rng(71)
    q = r.standard_normal((N, S, Nh, D), dtype=np.float32)
    k = r.standard_normal((N, Nkv, SLOTS, D), dtype=np.float32)
    v = r.standard_normal((N, Nkv, SLOTS, D), dtype=np.float32)
    dkf, kf = _kv(k, kt)
    dvf, vf = _kv(v, kt)
    sl = (slice(None), slice(None), slice(0, S))
    dk = ops.Q8(dkf.data[sl]) if kt == "q8_0" else dkf[sl]
    dv = ops.Q8(dvf.data[sl]) if kt == "q8_0" else dvf[sl]
    kf, vf = kf[:, :, :S], vf[:, :, :S]
    i = np.arange(S)
    m = np.broadcast_to(np.where(i[None, :] <= i[:, None], 0.0, -np.inf).astype(np.float32), (N, 1, S, S))
    dm, mf = _mask_dev(np.ascontiguousarray(m))
    dq = to_dev(q).permute(0, 2, 1, 3)                            # (N, Nh, S, D) view
    y = to_np(ops.flash_attn_ext(dq, dk, dv, dm, 1.0 / np.sqrt(D)))  # (N, S, Nh, D)
    assert _uses_mfma(kt, D, S, Nh, Nkv, S, mf) == "prefill"
    qs = np.unique(np.r_[0, 1, 31, 32, 63, 64, 65, 127, 128, 129, 511, 512, 1023, 1024, 1500, 2015, 2016, 2046, 2047,
                         r.integers(0, S, 17)])
    qf = np.ascontiguousarray(q[:, qs].transpose(0, 2, 1, 3))     # (N, Nh, len(qs), D)
    ms = np.ascontiguousarray(mf[:, :, qs])
    ref = orc.flash_attn_ext(qf, kf, vf, ms, 1.0 / np.sqrt(D), kt)
    _check(y[:, qs], ref, fa_bound(qf, kf, vf, ms, 1.0 / np.sqrt(D), kt, "prefill"))
    assert np.isfinite(y).all()
