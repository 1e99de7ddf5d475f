"""The tolerance helpers themselves (CPU): the bars must accept what they
state and reject what they state."""
import numpy as np
import pytest

from helpers import assert_bf16_ulp, assert_f32_close, rel_err
from oracle import oracle as orc


def test_bf16_bar_ulp_and_row_floor():
    ref = np.ones((4, 128), np.float32)
    ref[0, 5] = 1.2e-7                    # a cancelled output in a row of RMS ~1
    got = ref.copy()
    got[0, 5] = 1.8e-7                    # |diff| 6e-8 = 6e-8 of the row RMS, but many bf16 ulps
    rb, gb = orc.f32_to_bf16(ref), orc.f32_to_bf16(got)
    with pytest.raises(AssertionError):
        assert_bf16_ulp(gb, rb)
    assert_bf16_ulp(gb, rb, row_floor=True)
    got[1, 7] = 1.0 + 2 ** -6               # 2 bf16 ulps on a value of the row's own size
    with pytest.raises(AssertionError):
        assert_bf16_ulp(orc.f32_to_bf16(got), rb, row_floor=True)
    one_ulp = ref.copy()
    one_ulp[2, 3] = 1.0 + 2 ** -7
    assert_bf16_ulp(orc.f32_to_bf16(one_ulp), rb)


def test_f32_bar_relative_and_row_floor():
    ref = np.full((2, 64), 2.0, np.float32)
    ref[0, 0] = 1e-9
    got = ref.copy()
    got[0, 0] = 1e-9 + 1e-6               # 1e6 relative, 5e-7 of the row RMS
    assert rel_err(got, ref) > 1
    assert_f32_close(got, ref, row_floor=True)
    got[1, 1] = 2.0 * (1 + 3e-5)
    with pytest.raises(AssertionError):
        assert_f32_close(got, ref, row_floor=True)
