"""GPU parity: the other sampler steps on the device -- SDE ancestral
(mi_flow_step_sde), STORK4 (mi_stork4_step) and DCW (mi_dcw) -- and the
resident loop with them, against the oracle.
Bars, written here: every step does the reference's fp32 (and, for the
three-point derivative, double) operations in its order without contraction,
so results are bit-exact. The one reduction, STORK4's sums of squares for the
derivative guards, is summed in a different order than the oracle's; it only
decides the derivative order, and the inputs here sit far from the guard
thresholds, so the decisions agree and the results stay bit-exact.
STORK4 runs with synthetic ROCK4 tables of the reference's layout
(tests/rock4_tables.py), which steer every path, and with the reference's own
tables (solver-stork4-constants.h, kept as the fixture
tests/golden/rock4_reference.npz and pinned by the fourth-order conditions in
tests/test_rock4_reference_cpu.py)."""
import numpy as np
import pytest
from helpers import to_dev, to_np
from oracle import oracle as orc
from rock4_tables import degree_of, make_tables, reference_tables

from acestep_ops import ops
from acestep_ops import sampler as smp
from acestep_ops.device import DTensor

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(2, 300, 64), (3, 7, 5)])
def test_sde_step_bit_exact(dev, shape):
    print(f"sde step {shape}", flush=True)
    r = np.random.default_rng(11)
    x = r.standard_normal(shape).astype(np.float32)
    xd = to_dev(x)
    for tc, tn in ((1.0, 0.8), (0.8, 0.35), (0.35, 0.0)):
        v = r.standard_normal(shape).astype(np.float32)
        z = r.standard_normal(shape).astype(np.float32)
        smp.sde_step(to_dev(v), xd, to_dev(z), tc, tn)
        orc.sde_step(x, v, z, tc, tn)
        assert np.array_equal(to_np(xd), x)


def _stork_case(r, shape, kind):
    """velocities for one step: prev/prev2 shaped so the guards pick the order `kind` names"""
    v = r.standard_normal(shape).astype(np.float32)
    if kind == "order0":     # dv rms * h1 = 6 vt rms
        return v, (7.0 * v).astype(np.float32), (7.0 * v).astype(np.float32)
    if kind == "order1":     # d2v rms * h1^2 ~ 490 vt rms
        return v, (5.0 * v).astype(np.float32), (501.0 * v).astype(np.float32)
    p1 = (v + 0.05 * r.standard_normal(shape)).astype(np.float32)
    p2 = (p1 + 0.05 * r.standard_normal(shape)).astype(np.float32)
    return v, p1, p2


@pytest.mark.parametrize("shape", [(2, 300, 64), (3, 7, 5), (1, 1500, 64)])
@pytest.mark.parametrize("substeps", [10, 148])
def test_stork4_sequence_bit_exact(dev, shape, substeps):
    """Six steps from the bootstrap, history kept on the device, every derivative order."""
    print(f"stork4 sequence {shape} s={substeps}", flush=True)
    r = np.random.default_rng(12)
    tab = make_tables(21)
    tables = smp.Rock4Tables(*tab)
    x = r.standard_normal(shape).astype(np.float32)
    xd = to_dev(x)
    p1, p2 = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    pd, p2d = DTensor.zeros(shape, "f32"), DTensor.zeros(shape, "f32")
    ws = smp.stork4_workspace(xd)
    ts = [1.0, 0.9, 0.78, 0.66, 0.5, 0.31, 0.12]
    kinds = ["order2", "order2", "order0", "order1", "order2", "order2"]
    hist, h1, h2 = 0, 0.0, 0.0
    for k in range(len(ts) - 1):
        v, q1, q2 = _stork_case(r, shape, kinds[k])
        if k >= 2:  # steer the guards: overwrite the stored history on both sides
            p1[...], p2[...] = q1, q2
            pd, p2d = to_dev(q1), to_dev(q2)
        smp.stork4_step(to_dev(v), xd, ts[k], ts[k + 1], hist, h1, h2, pd, p2d, tables, ws, substeps)
        info = orc.stork4_step(x, v, ts[k], ts[k + 1], hist, h1, h2, p1, p2, substeps, tab)
        fb, order, deg = smp.stork4_status(ws)
        assert np.array_equal(to_np(xd), x), f"step {k}"
        assert np.array_equal(to_np(pd), p1) and np.array_equal(to_np(p2d), p2)
        assert (order, deg, fb) == (info[0], info[1], int(info[2])), f"step {k}: {(order, deg, fb)} vs {info}"
        hist = min(hist + 1, 2)
        h2, h1 = h1, float(np.float32(ts[k]) - np.float32(ts[k + 1]))


@pytest.mark.parametrize("substeps", [1, 10, 21, 100, 148, 400])
def test_stork4_reference_tables_bit_exact(dev, substeps):
    """Five steps from the bootstrap with the reference's ROCK4 tables: the
    degree each substep count selects (1 -> 2, 21 -> 22, 100 -> 105, 400 -> 148
    the largest), its real recurrence and finishing coefficients, bit-exact against
    the oracle, and the accepted degree as the reference's table lookup gives it."""
    print(f"stork4 reference tables s={substeps}", flush=True)
    r = np.random.default_rng(15)
    tab = reference_tables()
    tables = smp.Rock4Tables(*tab)
    shape = (2, 250, 64)
    x = r.standard_normal(shape).astype(np.float32)
    xd = to_dev(x)
    p1, p2 = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    pd, p2d = DTensor.zeros(shape, "f32"), DTensor.zeros(shape, "f32")
    ws = smp.stork4_workspace(xd)
    ts = [1.0, 0.93, 0.8, 0.62, 0.41, 0.2]
    hist, h1, h2 = 0, 0.0, 0.0
    for k in range(len(ts) - 1):
        v, _, _ = _stork_case(r, shape, "order2")
        smp.stork4_step(to_dev(v), xd, ts[k], ts[k + 1], hist, h1, h2, pd, p2d, tables, ws, substeps)
        info = orc.stork4_step(x, v, ts[k], ts[k + 1], hist, h1, h2, p1, p2, substeps, tab)
        fb, order, deg = smp.stork4_status(ws)
        assert np.array_equal(to_np(xd), x), f"step {k}"
        assert np.array_equal(to_np(pd), p1) and np.array_equal(to_np(p2d), p2)
        assert (order, deg, fb) == (info[0], info[1], int(info[2])), f"step {k}: {(order, deg, fb)} vs {info}"
        if k > 0:   # the bootstrap step is Euler (degree 0); later ones take the table's degree for
            # max(substeps, 2) (solver-stork.h:296)
            assert deg == degree_of(tab[0], max(substeps, 2))[0] and fb == 0
        hist = min(hist + 1, 2)
        h2, h1 = h1, float(np.float32(ts[k]) - np.float32(ts[k + 1]))


def test_stork4_nonfinite_fallbacks(dev):
    """an attempt that overflows is retried at half the substeps; when all do, Euler"""
    print("stork4 fallbacks", flush=True)
    r = np.random.default_rng(13)
    shape = (2, 64, 64)
    for tab, inf_at, want_deg, want_fb in ((make_tables(22, huge_from=8), None, 5, 0),
                                           (make_tables(22), 777, 0, 1)):
        x = r.standard_normal(shape).astype(np.float32)
        if inf_at is not None:
            x.reshape(-1)[inf_at] = np.inf
        v, p1, p2 = _stork_case(r, shape, "order2")
        xd, pd, p2d = to_dev(x), to_dev(p1), to_dev(p2)
        ws = smp.stork4_workspace(xd)
        smp.stork4_step(to_dev(v), xd, 0.5, 0.4, 2, 0.1, 0.1, pd, p2d, smp.Rock4Tables(*tab), ws, 10)
        info = orc.stork4_step(x, v, 0.5, 0.4, 2, 0.1, 0.1, p1, p2, 10, tab)
        fb, _, deg = smp.stork4_status(ws)
        assert (deg, fb) == (want_deg, want_fb) == (info[1], int(info[2]))
        assert np.array_equal(to_np(xd), x)


@pytest.mark.parametrize("t", [300, 7])
@pytest.mark.parametrize("mode", ["low", "high", "double", "pix"])
def test_dcw_bit_exact(dev, mode, t):
    print(f"dcw {mode} t={t}", flush=True)
    r = np.random.default_rng(14)
    x = r.standard_normal((2, t, 64)).astype(np.float32)
    v = r.standard_normal(x.shape).astype(np.float32)
    xd = to_dev(x)
    for tc, tn, s, sh in ((0.9, 0.7, 0.3, 0.2), (0.7, 0.4, 0.05, 0.0), (0.4, 0.2, 0.0, 0.0)):
        smp.dcw(mode, xd, to_dev(v), tc, tn, s, sh)
        orc.dcw(mode, x, v, tc, tn, s, sh)
        assert np.array_equal(to_np(xd), x)


@pytest.mark.parametrize("solver,dcw_mode", [("sde", None), ("stork4", None), ("euler", "low"),
                                             ("dpm3m", "double"), ("stork4", "high")])
def test_device_loop_other_solvers(dev, solver, dcw_mode):
    """The resident loop (guidance 1, so no APG reduction) with the velocity an
    affine map of x, against the same loop on the oracle: bit-exact."""
    print(f"device loop {solver} dcw={dcw_mode}", flush=True)
    r = np.random.default_rng(15)
    n, t, oc = 2, 120, 64
    noise = r.standard_normal((n, t, oc)).astype(np.float32)
    s1, b1 = (r.standard_normal(oc).astype(np.float32) * 0.3 for _ in range(2))
    ds1, db1 = to_dev(s1), to_dev(b1)
    sched = [1.0, 0.88, 0.75, 0.6, 0.45, 0.3, 0.18, 0.08]
    draws = [r.standard_normal(noise.shape).astype(np.float32) for _ in sched]
    ddraws = [to_dev(z) for z in draws]
    tab = make_tables(23)
    kw = dict(noise_fn=lambda k: ddraws[k], rock4=smp.Rock4Tables(*tab))
    if dcw_mode:
        kw.update(dcw_mode=dcw_mode, dcw_scaler=0.2, dcw_high_scaler=0.1)
    y = to_np(smp.DeviceSampler(to_dev(noise), sched, 1.0, solver, **kw).run(
        lambda x, _t: (ops.modulate(x, ds1, db1), None)))

    x = noise.copy()
    prev, prev2 = np.zeros_like(x), np.zeros_like(x)
    hist, h1, h2 = 0, 0.0, 0.0
    for k, tc in enumerate(sched):
        vt = ((x * (s1 + np.float32(1.0))).astype(np.float32) + b1).astype(np.float32)
        if k == len(sched) - 1:
            ref = orc.flow_final(x, vt, tc)
            break
        tn = sched[k + 1]
        if solver == "sde":
            orc.sde_step(x, vt, draws[k], tc, tn)
        elif solver == "stork4":
            orc.stork4_step(x, vt, tc, tn, hist, h1, h2, prev, prev2, 10, tab)
            h2, h1 = h1, float(np.float32(tc) - np.float32(tn))
        else:
            orc.flow_step(solver, x, vt, tc, tn, hist, prev, prev2)
        hist = min(hist + 1, 2)
        if dcw_mode:
            orc.dcw(dcw_mode, x, vt, tc, tn, 0.2, 0.1)
    assert np.array_equal(y, ref)
