"""Pinning the oracle's other sampler steps (orc_sde_step, orc_stork4_step,
orc_dcw) by closed forms and invariants, not by restating their loops:
  SDE: t_next = 0 gives the x0 prediction xt - vt t_curr exactly; t_next = 1
  gives the noise exactly; otherwise the float64 interpolation within a few ulp.
  STORK4: the bootstrap step is Euler exactly; a hand-derived degree-2 step;
  a constant velocity moves x by -dt (A_m + sum fpb) v with A_m the
  recurrence's weight, i.e. exactly -dt v for consistent tables; a velocity
  linear in t (any step sizes) makes the extrapolated stage velocities exact,
  so the step equals the scheme evaluated with the true v(t) at its stage
  times; a quadratic one gives the closed-form extrapolation
  v + (b + c h1) d + c d^2; the derivative guards and the halving/Euler
  fallback on non-finite results; the history rotation.
  DCW: zero scaler is the identity; denoised == xt is the Haar round trip
  (within an ulp); each band mode against an orthonormal Haar matrix in
  float64 (odd T zero-padded); "double" with a zero high scaler equals "low"
  bit for bit; pix in closed form.
Planting each of these mistakes in a copy of the oracle fails at least one
test: t_curr and t_next swapped in the SDE step; Y_{j-1} and Y_{j-2} swapped
in the recurrence; temp2 = 1 + temp3; the first stage from Y_{j-2}; h1 and h2
swapped in the three-point formula; the Taylor half factor dropped; the dv
guard's 5 as 0.5; the fallback halving skipped; the Haar high band with a + b;
the low band moved by (yL - xL).
"""
import numpy as np
import pytest
from oracle import oracle as orc
from rock4_tables import chain_weight, degree_of, make_tables


def _rng(seed):
    return np.random.default_rng(seed)


def _ulp(a):
    return np.spacing(np.abs(a).astype(np.float32)).astype(np.float64)


# ---- SDE ---------------------------------------------------------------------
def test_sde_endpoints_and_interpolation():
    r = _rng(1)
    x = r.standard_normal((2, 40, 8)).astype(np.float32)
    v = r.standard_normal(x.shape).astype(np.float32)
    z = r.standard_normal(x.shape).astype(np.float32)
    y = x.copy()
    orc.sde_step(y, v, z, 0.7, 0.0)
    assert np.array_equal(y, orc.flow_final(x, v, 0.7))
    y = x.copy()
    orc.sde_step(y, v, z, 0.7, 1.0)
    assert np.array_equal(y, z)
    y = x.copy()
    orc.sde_step(y, v, z, 0.8, 0.55)
    want = 0.55 * z.astype(np.float64) + 0.45 * (x.astype(np.float64) - 0.8 * v.astype(np.float64))
    assert np.all(np.abs(y - want) <= 4 * _ulp(want) + 1e-7)


# ---- STORK4 ------------------------------------------------------------------
def _stork(x, v, tc, tn, hist, h1, h2, p1, p2, s, tab):
    y, a, b = x.copy(), p1.copy(), p2.copy()
    info = orc.stork4_step(y, v, tc, tn, hist, h1, h2, a, b, s, tab)
    return y, a, b, info


def test_stork_bootstrap_is_euler_and_rotates_history():
    r = _rng(2)
    tab = make_tables(1)
    x = r.standard_normal(500).astype(np.float32)
    v = r.standard_normal(500).astype(np.float32)
    p1, p2 = r.standard_normal(500).astype(np.float32), r.standard_normal(500).astype(np.float32)
    y, a, b, info = _stork(x, v, 1.0, 0.9, 0, 0.0, 0.0, p1, p2, 10, tab)
    e = x.copy()
    orc.flow_step("euler", e, v, 1.0, 0.9)
    assert np.array_equal(y, e) and info == (0, 0, False)
    assert np.array_equal(a, v) and np.array_equal(b, p2)  # one record: prev2 untouched
    y, a, b, _ = _stork(x, v, 0.9, 0.8, 1, 0.1, 0.0, p1, p2, 10, tab)
    assert np.array_equal(a, v) and np.array_equal(b, p1)


def test_stork_degree_two_by_hand():
    """ms = [2]: Y1 = x - dt r0 v; Y2 = -dt mu v + (1 + k) Y1 - k x;
    out = Y2 - dt (b0 + b1 + b2 + b3) v, for a constant velocity (dv = 0)."""
    r0, mu, k = 0.3, 0.2, 0.6
    fpb = np.array([[0.1, 0.2, 0.05, 0.15]])
    tab = (np.array([2], np.int32), np.zeros((1, 6)), fpb, np.array([r0, mu, k]))
    x = np.linspace(-2, 2, 64).astype(np.float32)
    v = np.cos(np.arange(64)).astype(np.float32)
    dt = float(np.float32(0.7) - np.float32(0.5))
    y, _, _, info = _stork(x, v, 0.7, 0.5, 1, 0.2, 0.0, v, v, 2, tab)
    x64, v64 = x.astype(np.float64), v.astype(np.float64)
    y1 = x64 - dt * r0 * v64
    y2 = -dt * mu * v64 + (1 + k) * y1 - k * x64
    want = y2 - dt * fpb.sum() * v64
    assert info[1] == 2 and not info[2]
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-6)


@pytest.mark.parametrize("s", [2, 5, 10, 37, 148, 500])
def test_stork_constant_velocity(s):
    """v the same at every step: dv = d2v = 0 exactly, every stage velocity is v."""
    r = _rng(3)
    tab = make_tables(2, consistent=False)
    x = r.standard_normal(300).astype(np.float32)
    v = r.standard_normal(300).astype(np.float32)
    tc, tn = 0.8, 0.65
    dt = float(np.float32(tc) - np.float32(tn))
    y, _, _, info = _stork(x, v, tc, tn, 2, dt, dt, v, v, s, tab)
    m, row, off = degree_of(tab[0], s)
    a = chain_weight(tab[3][off:off + 2 * m - 1]) + tab[2][row].sum()
    assert info[1] == m
    want = x.astype(np.float64) - dt * a * v.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=0, atol=2e-6 * m)
    ms, fpa, fpb, recf = make_tables(2, consistent=True)
    y, _, _, _ = _stork(x, v, tc, tn, 2, dt, dt, v, v, s, (ms, fpa, fpb, recf))
    np.testing.assert_allclose(y, x.astype(np.float64) - dt * v.astype(np.float64), rtol=0, atol=2e-6 * m)


def _scheme_exact(x, vfun, tc, tn, s, tab):
    """The ROCK stage recurrence and finishing blend in float64 with the true
    velocity v(t) at each stage time (stage times advance like the stages)."""
    ms, fpa, fpb, recf = tab
    m, row, off = degree_of(ms, s)
    b = recf[off:off + 2 * m - 1]
    dt = float(np.float32(tc) - np.float32(tn))
    y2 = x.astype(np.float64)
    y1 = y2 - dt * b[0] * vfun(tc)
    c_prev, c = tc, tc - dt * b[0]
    for j in range(2, m + 1):
        mu, k = b[2 * (j - 2) + 1], b[2 * (j - 2) + 2]
        y1, y2 = -dt * mu * vfun(c) + (1 + k) * y1 - k * y2, y1
        c, c_prev = -dt * mu + (1 + k) * c - k * c_prev, c
    a = -dt * fpa[row]
    t2, t3, t4 = c + a[0], c + a[1] + a[2], c + a[3] + a[4] + a[5]
    w = -dt * fpb[row]
    return y1 + w[0] * vfun(c) + w[1] * vfun(t2) + w[2] * vfun(t3) + w[3] * vfun(t4)


@pytest.mark.parametrize("hist,h1,h2", [(1, 0.15, 0.0), (2, 0.15, 0.1), (2, 0.05, 0.2)])
def test_stork_linear_in_time_is_exact(hist, h1, h2):
    """v(t) = a + g (t - t_curr): the forward difference is g and the three-point
    second derivative 0 whatever h1 and h2 are, so the Taylor stage velocities
    are exact."""
    r = _rng(4)
    tab = make_tables(3)
    n = 400
    a0 = r.standard_normal(n)
    g = r.standard_normal(n) * 0.5
    x = r.standard_normal(n).astype(np.float32)
    tc, tn = 0.6, 0.45
    vf = lambda t: a0 + g * (t - tc)  # noqa: E731
    v = vf(tc).astype(np.float32)
    p1 = vf(tc + h1).astype(np.float32)
    p2 = vf(tc + h1 + h2).astype(np.float32)
    vf32 = lambda t: v.astype(np.float64) + g * (t - tc)  # noqa: E731  (v rounded as the oracle sees it)
    y, _, _, info = _stork(x, v, tc, tn, hist, h1, h2, p1, p2, 10, tab)
    assert info[0] == hist
    np.testing.assert_allclose(y, _scheme_exact(x, vf32, tc, tn, 10, tab), rtol=0, atol=3e-5)


def test_stork_quadratic_extrapolation():
    """v(t) = a + b d + c d^2 (d = t - t_curr): dv = b + c h1 (forward
    difference) and d2v = 2c (three-point), so the stage velocity is
    a + (b + c h1) d + c d^2."""
    r = _rng(5)
    tab = make_tables(4)
    n = 300
    a0, b0, c0 = r.standard_normal(n), r.standard_normal(n) * 0.5, r.standard_normal(n) * 0.5
    tc, tn, h1, h2 = 0.5, 0.4, 0.1, 0.15
    vf = lambda t: a0 + b0 * (t - tc) + c0 * (t - tc) ** 2  # noqa: E731
    v, p1, p2 = (vf(t).astype(np.float32) for t in (tc, tc + h1, tc + h1 + h2))
    x = r.standard_normal(n).astype(np.float32)
    y, _, _, info = _stork(x, v, tc, tn, 2, h1, h2, p1, p2, 10, tab)
    assert info[0] == 2
    ext = lambda t: a0 + (b0 + c0 * h1) * (t - tc) + c0 * (t - tc) ** 2  # noqa: E731
    np.testing.assert_allclose(y, _scheme_exact(x, ext, tc, tn, 10, tab), rtol=0, atol=5e-5)


def test_stork_guards():
    r = _rng(6)
    tab = make_tables(5)
    n = 256
    x = r.standard_normal(n).astype(np.float32)
    v = r.standard_normal(n).astype(np.float32)
    h = 0.1
    # dv rms * h1 = 6 * vt rms > 5 vt rms: no derivative, every stage uses v
    p1 = (v + 6.0 * v).astype(np.float32)
    y, _, _, info = _stork(x, v, 0.5, 0.4, 2, h, h, p1, p1, 10, tab)
    assert info[0] == 0
    np.testing.assert_allclose(y, _scheme_exact(x, lambda t: v.astype(np.float64), 0.5, 0.4, 10, tab), atol=2e-5)
    # 4 * vt rms passes the first guard
    p1 = (v + 4.0 * v).astype(np.float32)
    assert _stork(x, v, 0.5, 0.4, 1, h, 0.0, p1, p1, 10, tab)[3][0] == 1
    # d2v rms * h1^2 > 5 vt rms: first order only
    p2 = (v + 500.0 * v).astype(np.float32)
    assert _stork(x, v, 0.5, 0.4, 2, h, h, p1, p2, 10, tab)[3][0] == 1
    # h1 == 0: no derivative; h2 == 0: first order at most
    assert _stork(x, v, 0.5, 0.4, 2, 0.0, h, p1, p1, 10, tab)[3][0] == 0
    assert _stork(x, v, 0.5, 0.4, 2, h, 0.0, v, v, 10, tab)[3][0] == 1


def test_stork_nonfinite_fallbacks():
    r = _rng(7)
    x = r.standard_normal(128).astype(np.float32)
    v = r.standard_normal(128).astype(np.float32)
    # degrees >= 8 overflow: s = 10 fails, s = 5 succeeds
    tab = make_tables(6, huge_from=8)
    y, _, _, info = _stork(x, v, 0.5, 0.4, 2, 0.1, 0.1, v, v, 10, tab)
    assert info[1] == 5 and not info[2] and np.all(np.isfinite(y))
    y5, _, _, _ = _stork(x, v, 0.5, 0.4, 2, 0.1, 0.1, v, v, 5, tab)
    assert np.array_equal(y, y5)
    # an infinite latent makes every attempt non-finite (inf - inf): Euler
    tab = make_tables(6)
    x[3] = np.inf
    y, _, _, info = _stork(x, v, 0.5, 0.4, 2, 0.1, 0.1, v, v, 10, tab)
    e = x.copy()
    orc.flow_step("euler", e, v, 0.5, 0.4)
    assert info[2] and info[1] == 0 and np.array_equal(y, e)


# ---- DCW ---------------------------------------------------------------------
def _haar(t):
    """orthonormal analysis rows: low band (pairs summed), high band (differenced);
    an odd last frame is zero-padded"""
    tl = (t + 1) // 2
    lo, hi = np.zeros((tl, t)), np.zeros((tl, t))
    k = 1 / np.sqrt(2)
    for l in range(tl):
        lo[l, 2 * l] = hi[l, 2 * l] = k
        if 2 * l + 1 < t:
            lo[l, 2 * l + 1], hi[l, 2 * l + 1] = k, -k
    return lo, hi


def _dcw64(mode, x, v, tc, tn, s, sh):
    n, t, oc = x.shape
    lo, hi = _haar(t)
    out = np.empty(x.shape)
    for b in range(n):
        xb = x[b].astype(np.float64)
        db = xb - v[b].astype(np.float64) * np.float32(tn)
        if mode == "pix":
            out[b] = xb + s * (xb - db)
            continue
        xl, xh, yl, yh = lo @ xb, hi @ xb, lo @ db, hi @ db
        sl = tc * s if mode in ("low", "double") else 0.0
        shh = (1 - tc) * s if mode == "high" else (1 - tc) * sh if mode == "double" else 0.0
        xl, xh = xl + sl * (xl - yl), xh + shh * (xh - yh)
        # synthesis: the transposed rows; the zero-padded frame is dropped
        out[b] = lo.T @ xl + hi.T @ xh
    return out


@pytest.mark.parametrize("t", [64, 7])
@pytest.mark.parametrize("mode", ["low", "high", "double", "pix"])
def test_dcw_against_haar_matrix(mode, t):
    r = _rng(8)
    x = r.standard_normal((2, t, 6)).astype(np.float32)
    v = r.standard_normal(x.shape).astype(np.float32)
    y = x.copy()
    orc.dcw(mode, y, v, 0.7, 0.6, 0.4, 0.25)
    np.testing.assert_allclose(y, _dcw64(mode, x, v, 0.7, 0.6, 0.4, 0.25), rtol=0, atol=3e-6)


def test_dcw_identities():
    r = _rng(9)
    x = r.standard_normal((1, 32, 8)).astype(np.float32)
    v = r.standard_normal(x.shape).astype(np.float32)
    for mode in ("low", "high", "double", "pix"):
        y = x.copy()
        orc.dcw(mode, y, v, 0.5, 0.4, 0.0, 0.0)
        assert np.array_equal(y, x)
    # denoised == xt (t_next = 0): the bands do not move; the round trip is within an ulp
    y = x.copy()
    orc.dcw("low", y, v, 0.5, 0.0, 0.3)
    pair = np.abs(x).reshape(1, 16, 2, 8).max(axis=2).repeat(2, axis=1)  # a frame and its partner
    assert np.all(np.abs(y - x) <= 2 * _ulp(pair))
    # double with no high scaler is low; unknown modes act as low
    a, b, c = x.copy(), x.copy(), x.copy()
    orc.dcw("low", a, v, 0.5, 0.4, 0.3)
    orc.dcw("double", b, v, 0.5, 0.4, 0.3, 0.0)
    orc.dcw("bogus", c, v, 0.5, 0.4, 0.3)
    assert np.array_equal(a, b) and np.array_equal(a, c)
