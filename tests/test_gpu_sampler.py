"""GPU parity: the sampler's step math on the device (mi_apg_forward,
mi_flow_step, mi_flow_final) and the resident loop (acestep_ops.sampler.
DeviceSampler) against the oracle.
Bars, written here: the solvers and the final step do the reference's fp32
operations in its order, without contraction -> bit-exact. APG runs in
double like the reference, but sums the frames in a different order (a
parallel reduction): its double results differ in the last bits, so the
float output is within 1 ulp of the oracle's. The loop compounds those ulps
over steps: 1e-5 relative (plus 1e-6 absolute) after 8 steps."""
import numpy as np
import pytest
from helpers import to_dev, to_np
from oracle import oracle as orc

from acestep_ops import ops
from acestep_ops.device import DTensor
from acestep_ops import sampler as smp

pytestmark = pytest.mark.gpu


def _ulps(y, ref):
    return np.abs(y.astype(np.float64) - ref) / np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)


@pytest.mark.parametrize("n,t,oc", [(2, 300, 64), (1, 1000, 64), (3, 7, 5), (1, 50, 1024)])
def test_apg_two_steps(dev, n, t, oc):
    """Two consecutive calls (momentum), guidance 7 with the clip active on some
    channels (large differences) and not on others."""
    print(f"apg n={n} t={t} oc={oc}", flush=True)
    r = np.random.default_rng(n * 7 + t + oc)
    ra = np.zeros((n, t, oc))
    mb = None
    for step in range(2):
        cond = r.standard_normal((n, t, oc)).astype(np.float32)
        scale = np.where(np.arange(oc) % 2 == 0, 0.3, 0.01).astype(np.float32)
        unc = (cond - scale * r.standard_normal((n, t, oc))).astype(np.float32)
        dc, du = to_dev(cond), to_dev(unc)
        if mb is None:
            mb = smp.apg_buffer(dc)
        y = to_np(smp.apg_forward(dc, du, 7.0, mb, step == 0))
        ref = orc.apg_forward(cond, unc, 7.0, ra, step == 0)
        assert np.max(_ulps(y, ref)) <= 1.0


@pytest.mark.parametrize("solver", ["euler", "dpm3m"])
def test_solver_steps_bit_exact(dev, solver):
    print(f"flow step {solver}", flush=True)
    r = np.random.default_rng(3)
    shape = (2, 123, 64)
    x = r.standard_normal(shape).astype(np.float32)
    xd = to_dev(x)
    pd, p2d = DTensor.zeros(shape, "f32"), DTensor.zeros(shape, "f32")
    prev, prev2 = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    ts = [1.0, 0.87, 0.7, 0.41, 0.2, 0.05]
    hist = 0
    for k in range(len(ts) - 1):
        v = r.standard_normal(shape).astype(np.float32)
        smp.flow_step(solver, to_dev(v), xd, ts[k], ts[k + 1], hist, pd, p2d)
        orc.flow_step(solver, x, v, ts[k], ts[k + 1], hist, prev, prev2)
        hist = min(hist + 1, 2)
        assert np.array_equal(to_np(xd), x)
        if solver == "dpm3m":
            assert np.array_equal(to_np(pd), prev) and np.array_equal(to_np(p2d), prev2)
    v = r.standard_normal(shape).astype(np.float32)
    assert np.array_equal(to_np(smp.flow_final(xd, to_dev(v), 0.05)), orc.flow_final(x, v, 0.05))


@pytest.mark.parametrize("solver,guidance", [("euler", 4.0), ("dpm3m", 4.0), ("euler", 1.0)])
def test_device_loop(dev, solver, guidance):
    """The whole loop on the device with a model whose velocities are per-channel
    affine maps of x (the AdaLN modulate op), against the same loop on the oracle."""
    print(f"device loop {solver} cfg={guidance}", flush=True)
    r = np.random.default_rng(4)
    n, t, oc = 2, 200, 64
    noise = r.standard_normal((n, t, oc)).astype(np.float32)
    s1, b1, s2, b2 = (r.standard_normal(oc).astype(np.float32) * 0.3 for _ in range(4))
    d = {k: to_dev(v) for k, v in (("s1", s1), ("b1", b1), ("s2", s2), ("b2", b2))}
    sched = [1.0, 0.9, 0.75, 0.6, 0.45, 0.3, 0.18, 0.08]

    def model(x, _t):
        return ops.modulate(x, d["s1"], d["b1"]), ops.modulate(x, d["s2"], d["b2"])

    y = to_np(smp.DeviceSampler(to_dev(noise), sched, guidance, solver).run(model))

    def mod(x, s, b):
        return ((x * (s + np.float32(1.0))).astype(np.float32) + b).astype(np.float32)

    x = noise.copy()
    ra = np.zeros(x.shape)
    prev, prev2 = np.zeros_like(x), np.zeros_like(x)
    hist = 0
    for k, tc in enumerate(sched):
        vc, vu = mod(x, s1, b1), mod(x, s2, b2)
        vt = orc.apg_forward(vc, vu, guidance, ra, k == 0) if guidance > 1 else vc
        if k == len(sched) - 1:
            ref = orc.flow_final(x, vt, tc)
        else:
            orc.flow_step(solver, x, vt, tc, sched[k + 1], hist, prev, prev2)
            hist = min(hist + 1, 2)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)
    if guidance <= 1:
        assert np.array_equal(y, ref)  # no APG: every op is bit-exact
