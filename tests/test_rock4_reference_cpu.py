"""The reference's ROCK4 tables (fixture tests/golden/rock4_reference.npz, read
from solver-stork4-constants.h by tests/golden/make_rock4_tables.py), pinned
by what ROCK4 is: for every one of the 50 degrees, the recurrence and the
finishing procedure together integrate y' = lambda y to fourth order, so the
stability polynomial's first five coefficients are 1, 1, 1/2, 1/6, 1/24
(Abdulle 2002). One misread, misplaced or dropped coefficient breaks this; the
planted mistakes below show that it does."""
import numpy as np
import pytest

from rock4_tables import degree_of, reference_tables, stability_polynomial

TAYLOR = np.array([1.0, 1.0, 1.0 / 2, 1.0 / 6, 1.0 / 24])


def _order4_error(tab, row):
    r = stability_polynomial(*tab, row)
    return float(np.max(np.abs(r[:5] - TAYLOR) / TAYLOR))


def test_reference_tables_shape():
    ms, fpa, fpb, recf = reference_tables()
    assert ms.shape == (50,) and fpa.shape == (50, 6) and fpb.shape == (50, 4) and recf.shape == (4382,)
    assert ms[0] == 1 and ms[-1] == 148 and np.all(np.diff(ms) > 0)
    assert int(np.sum(2 * ms.astype(np.int64) - 1)) == recf.size
    assert degree_of(ms, 21) == (22, 20, int(np.sum(2 * ms[:20] - 1)))
    assert degree_of(ms, 500)[0] == 148


def test_every_degree_is_fourth_order():
    tab = reference_tables()
    worst = max(_order4_error(tab, row) for row in range(len(tab[0])))
    assert worst < 1e-12, worst


@pytest.mark.parametrize("plant", ["swap_recf", "drop_fpa", "shift_fpb", "recf_sign"])
def test_planted_table_mistakes_break_the_order(plant):
    ms, fpa, fpb, recf = (a.copy() for a in reference_tables())
    row = 30                                  # degree 44
    off = degree_of(ms, int(ms[row]))[2]
    if plant == "swap_recf":
        recf[off + 3], recf[off + 4] = recf[off + 4], recf[off + 3]
    elif plant == "drop_fpa":
        fpa[row, 4] = 0.0
    elif plant == "shift_fpb":
        fpb[row] = np.roll(fpb[row], 1)
    else:
        recf[off + 10] = -recf[off + 10]
    assert _order4_error((ms, fpa, fpb, recf), row) > 1e-6
