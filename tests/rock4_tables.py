"""Synthetic ROCK4 coefficient tables for the STORK4 tests.

The reference's tables (solver-stork4-constants.h: Abdulle's ROCK4 degrees,
finishing and recurrence coefficients) are caller data of mi_stork4_step; the
step's arithmetic does not depend on their values, so the tests use tables of
the same shape and layout built here:
  ms    ascending degrees;
  recf  per degree m a block of 2m - 1 values: the first stage's weight, then
        (mu_j, kappa_j) for j = 2..m -- the stage is
        Y_j = -dt mu_j v + (1 + kappa_j) Y_{j-1} - kappa_j Y_{j-2};
  fpa   [len(ms)][6] finishing stage offsets, fpb [len(ms)][4] blend weights.
`consistent=True` sets each degree's last blend weight so that a constant
velocity integrates exactly (the weights of v sum to -dt), as a real ROCK4
table does.
"""
import os

import numpy as np

DEGREES = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 14, 16, 18, 20, 24, 28, 32, 40, 48, 64, 80, 100, 128, 148]


def chain_weight(recf_block) -> float:
    """A_m with Y_m = x - dt A_m v for a constant velocity (exact arithmetic)."""
    a_prev, a = 0.0, float(recf_block[0])
    for j in range(2, (len(recf_block) + 1) // 2 + 1):
        mu, kap = float(recf_block[2 * (j - 2) + 1]), float(recf_block[2 * (j - 2) + 2])
        a_prev, a = a, mu + (1.0 + kap) * a - kap * a_prev
    return a


def make_tables(seed=0, degrees=DEGREES, consistent=True, huge_from=None):
    """(ms, fpa, fpb, recf). huge_from: degrees >= this get kappa = 1e20 (their
    recurrence overflows), for the non-finite fallback tests."""
    r = np.random.default_rng(seed)
    ms = np.asarray(degrees, np.int32)
    blocks = []
    for m in ms:
        b = np.empty(2 * m - 1)
        b[0] = r.uniform(0.05, 0.3) / m
        b[1::2] = r.uniform(0.02, 0.2, m - 1) / m
        b[2::2] = r.uniform(0.3, 0.9, m - 1)
        if huge_from is not None and m >= huge_from:
            b[2::2] = 1e20  # |Y_j| grows ~1e20 per stage: overflows from the fourth stage
        blocks.append(b)
    recf = np.concatenate(blocks)
    fpa = r.uniform(-0.3, 0.6, (len(ms), 6))
    fpb = r.uniform(0.05, 0.3, (len(ms), 4))
    if consistent:
        for i, b in enumerate(blocks):
            fpb[i, 3] = 1.0 - chain_weight(b) - fpb[i, :3].sum()
    return ms, fpa, fpb, recf


def degree_of(ms, s):
    """(degree, row, recf offset) the substep count s selects: the smallest
    tabulated degree >= s (the largest when none is), its row, and the start of
    its recf block (the blocks of the smaller degrees come first)."""
    ms = np.asarray(ms)
    s = min(int(s), int(ms[-1]))
    row = int(np.searchsorted(ms, s, side="left"))
    off = int(np.sum(2 * ms[:row] - 1))
    return int(ms[row]), row, off


REFERENCE_NPZ = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rock4_reference.npz")


def reference_tables():
    """(ms, fpa, fpb, recf): the reference's own ROCK4 tables
    (solver-stork4-constants.h), from the fixture tests/golden/make_rock4_tables.py wrote."""
    d = np.load(REFERENCE_NPZ)
    return d["ms"], d["fpa"], d["fpb"], d["recf"]


def stability_polynomial(ms, fpa, fpb, recf, row):
    """Coefficients (float64, ascending powers of z = h*lambda) of the polynomial
    R with y_1 = R(z) y_0 when the degree-`row` scheme -- the recurrence
    Y_1 = Y_0 + mu_1 z Y_0, Y_j = mu_j z Y_{j-1} + (1 + kappa_j) Y_{j-1} - kappa_j Y_{j-2},
    then the four finishing stages and the fpb blend, as solver-stork.h:193-267
    applies them -- integrates y' = lambda y over one step h."""
    from numpy.polynomial import polynomial as P

    m = int(ms[row])
    off = int(np.sum(2 * np.asarray(ms[:row], np.int64) - 1))
    b = np.asarray(recf[off:off + 2 * m - 1], np.float64)
    z = [0.0, 1.0]
    y2, y1 = np.array([1.0]), np.array([1.0, b[0]])
    for j in range(2, m + 1):
        mu, kap = b[2 * (j - 2) + 1], b[2 * (j - 2) + 2]
        y2, y1 = y1, P.polyadd(P.polyadd(P.polymul([0.0, mu], y1), (1.0 + kap) * y1), -kap * y2)
    a, w = fpa[row], fpb[row]
    f1 = P.polymul(z, y1)
    f2 = P.polymul(z, P.polyadd(y1, a[0] * f1))
    f3 = P.polymul(z, P.polyadd(P.polyadd(y1, a[1] * f1), a[2] * f2))
    f4 = P.polymul(z, P.polyadd(P.polyadd(P.polyadd(y1, a[3] * f1), a[4] * f2), a[5] * f3))
    r = y1
    for c, f in zip(w, (f1, f2, f3, f4)):
        r = P.polyadd(r, c * f)
    return r
