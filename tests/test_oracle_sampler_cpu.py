"""Pinning the sampler oracle (orc_apg_forward, orc_flow_step, orc_flow_final)
by closed forms, not by restating its loops:
  APG: guidance scale 1 -> cond exactly; uncond == cond -> cond exactly; a
  per-channel difference orthogonal to cond -> cond + (scale - 1) diff, clipped
  to norm 2.5 when longer; a difference parallel to cond -> cond; the
  momentum recurrence ra = diff + m ra_prev.
  Solvers: a constant velocity integrates exactly (Euler and DPM++ 3M); on a
  uniform grid DPM++ 3M integrates a quadratic velocity exactly after its
  Euler and AB2 bootstrap steps, whose local errors are known in closed form.
Planting each of these mistakes in a copy of the oracle fails at least one
test: the projection normalized by the difference's norm instead of cond's, no clip, a clip
over channels instead of frames, the momentum sign flipped, AB3 weight 15/12
instead of 16/12, the history shift skipped, the final step with + instead
of -.
"""
import numpy as np
from oracle import oracle as orc


def _rng(seed):
    return np.random.default_rng(seed)


def test_apg_identities():
    r = _rng(1)
    cond = r.standard_normal((2, 50, 8)).astype(np.float32)
    unc = r.standard_normal((2, 50, 8)).astype(np.float32)
    ra = np.zeros(cond.shape)
    assert np.array_equal(orc.apg_forward(cond, unc, 1.0, ra, True), cond)
    ra = np.zeros(cond.shape)
    assert np.array_equal(orc.apg_forward(cond, cond, 7.0, ra, True), cond)


def _orthogonal(cond, seed, norm):
    """per channel (over frames) a vector orthogonal to cond[:, :, c] with the given norm"""
    r = _rng(seed)
    d = r.standard_normal(cond.shape)
    c = cond.astype(np.float64)
    d -= c * (np.sum(d * c, axis=1, keepdims=True) / np.sum(c * c, axis=1, keepdims=True))
    return d * (norm / np.linalg.norm(d, axis=1, keepdims=True))


def test_apg_orthogonal_difference_and_clip():
    cond = _rng(2).standard_normal((1, 64, 6)).astype(np.float32)
    for norm, scale in ((0.5, 3.0), (10.0, 4.0)):
        d = _orthogonal(cond, 3, norm)
        unc = (cond.astype(np.float64) - d).astype(np.float32)
        dd = cond.astype(np.float64) - unc.astype(np.float64)  # the difference as the oracle sees it
        ra = np.zeros(cond.shape)
        y = orc.apg_forward(cond, unc, scale, ra, True)
        nd = np.linalg.norm(dd, axis=1, keepdims=True)
        clip = np.minimum(1.0, 2.5 / nd)
        dc = dd * clip
        c = cond.astype(np.float64)
        orth = dc - c * (np.sum(dc * c, axis=1, keepdims=True) / np.sum(c * c, axis=1, keepdims=True))
        ref = c + (scale - 1.0) * orth
        np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-6)
        if norm > 2.5:  # the clip acted: the guidance added has norm (scale - 1) * 2.5 per channel
            g = y.astype(np.float64) - c
            np.testing.assert_allclose(np.linalg.norm(g, axis=1), (scale - 1.0) * 2.5, rtol=1e-5)


def test_apg_parallel_difference_is_dropped():
    cond = _rng(4).standard_normal((2, 40, 5)).astype(np.float32)
    unc = (cond * np.float32(0.25)).astype(np.float32)
    ra = np.zeros(cond.shape)
    y = orc.apg_forward(cond, unc, 5.0, ra, True)
    np.testing.assert_allclose(y, cond, rtol=1e-6, atol=1e-6)


def test_apg_momentum_recurrence():
    r = _rng(5)
    c1, u1, c2, u2 = (r.standard_normal((1, 30, 4)).astype(np.float32) for _ in range(4))
    ra = np.zeros(c1.shape)
    orc.apg_forward(c1, u1, 2.0, ra, True)
    d1 = c1.astype(np.float64) - u1.astype(np.float64)
    assert np.array_equal(ra, d1)
    orc.apg_forward(c2, u2, 2.0, ra, False, momentum=-0.75)
    d2 = c2.astype(np.float64) - u2.astype(np.float64)
    assert np.array_equal(ra, d2 + (-0.75) * d1)


def _run(solver, v_of_t, ts, x0):
    x = x0.copy()
    prev = np.zeros_like(x)
    prev2 = np.zeros_like(x)
    hist = 0
    for k in range(len(ts) - 1):
        v = v_of_t(ts[k]).astype(np.float32)
        orc.flow_step(solver, x, v, float(ts[k]), float(ts[k + 1]), hist, prev, prev2)
        hist = min(hist + 1, 2)
    return x


def test_constant_velocity_integrates_exactly():
    x0 = _rng(6).standard_normal(1000).astype(np.float32)
    v = _rng(7).standard_normal(1000).astype(np.float32)
    ts = np.linspace(1.0, 0.0, 9).astype(np.float32)
    for solver in ("euler", "dpm3m"):
        x = _run(solver, lambda t: v, ts, x0)
        np.testing.assert_allclose(x, x0.astype(np.float64) - v.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_dpm3m_quadratic_velocity():
    """dx/dt = v(t) = a + b t + c t^2 backwards from t = 1 on a uniform grid of h:
    Euler's local error on the first step, AB2's on the second, none after."""
    a, b, c = 0.3, -1.1, 0.7
    n = 16
    h = 1.0 / n
    ts = np.array([1.0 - k * h for k in range(n + 1)], np.float64)
    v = lambda t: np.full(4, a + b * t + c * t * t)  # noqa: E731
    V = lambda t: a * t + b * t * t / 2 + c * t ** 3 / 3  # noqa: E731
    x = _run("dpm3m", lambda t: v(float(t)), ts.astype(np.float32), np.zeros(4, np.float32))
    exact = -(V(1.0) - V(0.0))
    # Euler step 1: x1 = -h v(t0); AB2 step 2: -h (1.5 v(t1) - 0.5 v(t0)); AB3 exact afterwards
    e1 = -h * v(ts[0])[0] + (V(ts[0]) - V(ts[1]))
    e2 = -h * (1.5 * v(ts[1])[0] - 0.5 * v(ts[0])[0]) + (V(ts[1]) - V(ts[2]))
    np.testing.assert_allclose(x, exact + e1 + e2, rtol=0, atol=2e-6)


def test_final_step():
    xt = _rng(8).standard_normal(100).astype(np.float32)
    vt = _rng(9).standard_normal(100).astype(np.float32)
    y = orc.flow_final(xt, vt, 0.25)
    assert np.array_equal(y, xt - vt * np.float32(0.25))
