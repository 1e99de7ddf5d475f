"""GPU parity, bit-exact: Q8_0 get_rows dequant, Q8_0 quantize (both ggml
rounding variants) through ggml_cpy and the batched KV-cache store, F16/BF16
cache writes, and the quantize -> get_rows round trip."""
import numpy as np
import pytest
from helpers import randn, rng, to_dev, to_np
from oracle import oracle as orc

from acestep_ops import Q8_0_CPU_X86, Q8_0_REF, ops
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu
VARIANTS = [(Q8_0_CPU_X86, "x86"), (Q8_0_REF, "ref")]


def _q8_table(n_rows, n, seed):
    return orc.quantize_q8_0(randn((n_rows, n), seed=seed, scale=0.02), "ref")


@pytest.mark.parametrize("n_rows,n,n_ids", [(4096, 1024, 512), (2048, 2048, 1000), (300, 2560, 64), (40, 8192, 33),
                                           (50, 96, 7)])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_get_rows_q8_0(dev, n_rows, n, n_ids, out):
    print(f"get_rows q8_0 {n_rows}x{n} ids={n_ids} out={out}", flush=True)
    tab = _q8_table(n_rows, n, seed=n)
    ids = rng(n_ids).integers(0, n_rows, n_ids).astype(np.int32)
    ids[:3] = [0, n_rows - 1, ids[2]]
    od = out
    y = to_np(ops.get_rows(ops.Q8(to_dev(tab, dev)), to_dev(ids, dev), out_dtype=od))
    ref = orc.get_rows(tab, orc.Q8_0, n, ids)
    if out == "bf16":
        ref = orc.f32_to_bf16(ref)
    assert np.array_equal(y.view(np.uint8), ref.view(np.uint8))


def test_get_rows_q8_0_all_codes_and_scales(dev):
    """Every int8 code against fp16 scales incl. 0, subnormals, max normal."""
    scales = np.array([0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x1E00, 0x7BFF, 0x8001, 0xBC00, 0x2E66], np.uint16)
    codes = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    rows = []
    for s in scales:
        row = np.zeros(8 * 34, np.uint8)
        for b in range(8):
            row[b * 34:b * 34 + 2] = np.frombuffer(s.tobytes(), np.uint8)
            row[b * 34 + 2:b * 34 + 34] = codes[b * 32:(b + 1) * 32].view(np.uint8)
        rows.append(row)
    tab = np.stack(rows)
    ids = np.arange(len(scales), dtype=np.int32)
    y = to_np(ops.get_rows(ops.Q8(to_dev(tab, dev)), to_dev(ids, dev)))
    ref = orc.get_rows(tab, orc.Q8_0, 256, ids)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("ttype", ["f32", "f16", "bf16"])
def test_get_rows_plain_tables(dev, ttype):
    n_rows, n = 1000, 1024
    t = randn((n_rows, n), seed=2)
    if ttype == "f16":
        host = orc.f32_to_f16(t)
        dt = to_dev(host, dev, f16=True)
        code = orc.F16
    elif ttype == "bf16":
        host = orc.f32_to_bf16(t)
        dt = to_dev(host, dev, bf16=True)
        code = orc.BF16
    else:
        host, dt, code = t, to_dev(t, dev), orc.F32
    ids = rng(3).integers(0, n_rows, 200).astype(np.int32)
    y = to_np(ops.get_rows(dt, to_dev(ids, dev)))
    assert np.array_equal(y, orc.get_rows(host, code, n, ids))


def test_get_rows_q8_0_waves_walk_several_ids(dev):
    """More ids than the LDS kernel's grid has waves (256 CUs x 16 workgroups x 4
    waves on this device): each wave walks several ids a grid stride apart, the
    next row in flight under the current stores; invalid ids among them count
    and give zero rows, and the valid ones stay bit-exact."""
    n_rows, n, n_ids = 512, 256, 70001
    tab = _q8_table(n_rows, n, seed=3)
    ids = rng(5).integers(0, n_rows, n_ids).astype(np.int32)
    bad = rng(6).choice(n_ids, 97, replace=False)
    ids[bad] = np.where(np.arange(bad.size) % 2 == 0, -3, n_rows + 7)
    err = DTensor.zeros((1,), "i32")
    y = to_np(ops.get_rows(ops.Q8(to_dev(tab, dev)), to_dev(ids, dev), err=err))
    assert int(err.item()) == bad.size
    good = np.ones(n_ids, bool)
    good[bad] = False
    assert np.array_equal(y[good], orc.get_rows(tab, orc.Q8_0, n, ids[good]))
    assert not y[bad].any()


def test_get_rows_out_of_range_ids(dev):
    tab = _q8_table(64, 256, seed=1)
    ids = np.array([0, 64, -1, 5, 1 << 30], np.int32)
    err = DTensor.zeros((1,), "i32")
    y = to_np(ops.get_rows(ops.Q8(to_dev(tab, dev)), to_dev(ids, dev), err=err))
    assert int(err.item()) == 3
    good = np.array([0, 3])
    assert np.array_equal(y[good], orc.get_rows(tab, orc.Q8_0, 256, ids[good]))
    assert not y[[1, 2, 4]].any()


@pytest.mark.parametrize("n,n_ids", [(32, 1), (64, 77), (128, 1025), (128, 4099), (160, 333)])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_get_rows_q8_0_short_rows(dev, n, n_ids, out):
    """Rows shorter than one wave-wide store (KV-cache heads) take the flat
    chunk-per-thread kernel: chunk counts that end mid-workgroup, strided ids,
    padded output rows, and invalid ids (zeros, counted once per row)."""
    print(f"get_rows q8_0 short rows n={n} ids={n_ids} out={out}", flush=True)
    n_rows = 700
    tab = _q8_table(n_rows, n, seed=n + n_ids)
    ids2 = rng(n_ids).integers(0, n_rows, (n_ids, 2)).astype(np.int32)
    bad = np.arange(n_ids) % 97 == 5
    ids2[bad, 0] = np.where(np.arange(bad.sum()) % 2 == 0, -3, n_rows)
    d_ids = to_dev(ids2, dev)[:, 0]  # ids with a stride of 2 elements
    pad = 8 if out == "f32" else 16
    yfull = DTensor.full_byte((n_ids, n + pad), 0x7F, "f32" if out == "f32" else "bf16")
    y = yfull[:, :n]
    err = DTensor.zeros((1,), "i32")
    ops.get_rows(ops.Q8(to_dev(tab, dev)), d_ids, out=y, out_dtype=out, err=err)
    got = to_np(yfull)
    ids = ids2[:, 0]
    ref = np.zeros((n_ids, n), np.float32)
    ref[~bad] = orc.get_rows(tab, orc.Q8_0, n, ids[~bad])
    if out == "bf16":
        ref = orc.f32_to_bf16(ref)
    assert np.array_equal(got[:, :n].view(np.uint8), ref.view(np.uint8))
    assert (got[:, n:].view(np.uint8) == 0x7F).all()  # padding untouched
    assert int(err.item()) == int(bad.sum())


def _tie_blocks():
    """Blocks separating the two quantizers: exact .5 ties under both id
    formulas, amax values where 127/amax != 1/(amax/127) in fp32, zero blocks,
    subnormal-scale blocks."""
    r = rng(11)
    blocks = []
    b = np.arange(32, dtype=np.float32) - 16.0  # amax 16 -> id = 127/16: x*id hits .5 at multiples of 16/127*?
    blocks.append(b)
    b = np.zeros(32, np.float32)
    b[0] = 127.0
    b[1:] = np.arange(1, 32, dtype=np.float32) + 0.5  # id = 1: exact halves 1.5, 2.5, ...
    blocks.append(b)
    b = -b.copy()
    blocks.append(b)
    blocks.append(np.zeros(32, np.float32))
    blocks.append((r.standard_normal(32) * 1e-6).astype(np.float32))     # fp16 d subnormal
    blocks.append((r.standard_normal(32) * 1e-10).astype(np.float32))    # d underflows to 0 in fp16
    blocks.append((r.standard_normal(32) * 60000).astype(np.float32))    # d near fp16 max
    # sweep amax so that 127/amax and 1/(amax/127) differ
    for k in range(57):
        amax = np.float32(1.0 + k * 0.0173)
        v = (r.uniform(-1, 1, 32) * amax).astype(np.float32)
        v[k % 32] = amax
        blocks.append(v)
    return np.stack(blocks)


@pytest.mark.parametrize("rounding,variant", VARIANTS)
@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_cpy_q8_0_bitexact(dev, rounding, variant, src):
    x = np.concatenate([_tie_blocks().reshape(-1), randn((64 * 128,), seed=4)]).reshape(-1, 128)
    if src == "bf16":
        xb = orc.f32_to_bf16(x)
        xs, xd = orc.bf16_to_f32(xb), to_dev(xb, dev, bf16=True)
    else:
        xs, xd = x, to_dev(x, dev)
    dst = DTensor.zeros((x.shape[0], 4 * 34), "u8")
    ops.cpy(xd, ops.Q8(dst), rounding=rounding)
    ref = orc.quantize_q8_0(xs, variant)
    assert np.array_equal(to_np(dst), ref)


@pytest.mark.parametrize("dst", ["f16", "bf16", "f32"])
def test_cpy_plain_types(dev, dst):
    x = randn((40, 128), seed=5) * 100
    out = DTensor.empty((40, 128), dst)
    ops.cpy(to_dev(x, dev), out)
    ref = {"f16": orc.f32_to_f16, "bf16": orc.f32_to_bf16, "f32": lambda a: a}[dst](x)
    assert np.array_equal(to_np(out), ref)


@pytest.mark.parametrize("rounding,variant", VARIANTS)
@pytest.mark.parametrize("B,T,decode", [(4, 64, False), (8, 1, True)])
def test_kv_store_q8_0(dev, rounding, variant, B, T, decode):
    """K,V [D, Nkv, T, B] -> Q8_0 caches [D, max_seq, Nkv, n_sets] at per-sequence slots,
    then dequantized back with get_rows. Untouched slots keep their sentinel."""
    print(f"kv_store B={B} T={T} {variant}", flush=True)
    D, Nkv, max_seq, n_sets = 128, 8, 512, B + 2
    r = rng(B * T)
    k = randn((B, T, Nkv, D), seed=1)
    v = randn((B, T, Nkv, D), seed=2)
    pos0 = r.integers(0, max_seq - T + 1, B).astype(np.int32)
    sets = r.permutation(n_sets)[:B].astype(np.int32)
    rb = D // 32 * 34
    kc = DTensor.full_byte((n_sets, Nkv, max_seq, rb), 0xA5)
    vc = DTensor.full_byte((n_sets, Nkv, max_seq, rb), 0x5A)
    ops.kv_store(to_dev(k, dev), ops.Q8(kc), to_dev(pos0, dev), v=to_dev(v, dev), v_cache=ops.Q8(vc),
                 sets=to_dev(sets, dev), rounding=rounding)
    kch, vch = to_np(kc), to_np(vc)
    written = np.zeros((n_sets, Nkv, max_seq), bool)
    for b in range(B):
        s, p = sets[b], pos0[b]
        written[s, :, p:p + T] = True
        for name, src, cache in (("k", k, kch), ("v", v, vch)):
            want = orc.quantize_q8_0(src[b].transpose(1, 0, 2), variant)  # (Nkv, T, rb)
            assert np.array_equal(cache[s, :, p:p + T], want), f"{name} b={b}"
    assert (kch[~written] == 0xA5).all() and (vch[~written] == 0x5A).all()
    # round trip: dequantize every written K row through get_rows
    flat = kc.view(-1, rb)
    ids = np.flatnonzero(written.reshape(-1)).astype(np.int32)
    y = to_np(ops.get_rows(ops.Q8(flat), to_dev(ids, dev)))
    assert np.array_equal(y, orc.dequantize_q8_0(kch.reshape(-1, rb)[ids]))


@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_kv_store_q8_0_tiles_with_bad_slots(dev, src):
    """Q8_0 caches written 8 consecutive slots of one head per wave tile, next
    to tiles that mix valid and out-of-range slots (the bad rows counted and
    skipped, the valid ones stored) and a sequence in a missing set."""
    print(f"kv_store q8_0 tiles + bad slots {src}", flush=True)
    D, Nkv, max_seq, B, T = 128, 8, 96, 3, 24
    k = randn((B, T, Nkv, D), seed=13)
    v = randn((B, T, Nkv, D), seed=14)
    if src == "bf16":
        kb, vb = orc.f32_to_bf16(k), orc.f32_to_bf16(v)
        k, v = orc.bf16_to_f32(kb), orc.bf16_to_f32(vb)
        kd, vd = to_dev(kb, dev, bf16=True), to_dev(vb, dev, bf16=True)
    else:
        kd, vd = to_dev(k, dev), to_dev(v, dev)
    rb = D // 32 * 34
    pos0 = np.array([5, max_seq - 20, 40], np.int32)  # sequence 1: slots past the end from t = 20
    sets = np.array([0, 2, 9], np.int32)              # set 9 does not exist
    kc = DTensor.full_byte((3, Nkv, max_seq, rb), 0xA5)
    vc = DTensor.full_byte((3, Nkv, max_seq, rb), 0x5A)
    err = DTensor.zeros((1,), "i32")
    ops.kv_store(kd, ops.Q8(kc), to_dev(pos0, dev), v=vd, v_cache=ops.Q8(vc), sets=to_dev(sets, dev), err=err)
    assert int(err.item()) == 2 * ((T - 20) * Nkv + T * Nkv)
    kch, vch = to_np(kc), to_np(vc)
    written = np.zeros((3, Nkv, max_seq), bool)
    for b, n in ((0, T), (1, 20)):
        s, p = sets[b], pos0[b]
        written[s, :, p:p + n] = True
        for src_, cache in ((k, kch), (v, vch)):
            want = orc.quantize_q8_0(src_[b, :n].transpose(1, 0, 2), "x86")
            assert np.array_equal(cache[s, :, p:p + n], want), f"b={b}"
    assert (kch[~written] == 0xA5).all() and (vch[~written] == 0x5A).all()


def test_kv_store_f16_cache_and_bad_slots(dev):
    """F16 cache (the Qwen3 LM's cache type) and out-of-range slots/sets."""
    D, Nkv, max_seq, B, T = 128, 8, 64, 3, 4
    k = randn((B, T, Nkv, D), seed=3)
    kc = DTensor.zeros((B, Nkv, max_seq, D), "f16")
    pos0 = np.array([0, 62, 10], np.int32)  # sequence 1 overruns max_seq at t >= 2
    sets = np.array([0, 1, 7], np.int32)    # set 7 does not exist
    err = DTensor.zeros((1,), "i32")
    ops.kv_store(to_dev(k, dev), kc, to_dev(pos0, dev), sets=to_dev(sets, dev), err=err)
    out = to_np(kc)
    assert int(err.item()) == (T - 2) * Nkv + T * Nkv
    assert np.array_equal(out[0, :, 0:T], orc.f32_to_f16(k[0].transpose(1, 0, 2)))
    assert np.array_equal(out[1, :, 62:64], orc.f32_to_f16(k[1, :2].transpose(1, 0, 2)))
    assert not out[2].any()
