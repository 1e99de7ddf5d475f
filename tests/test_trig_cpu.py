"""Host check of sincos_rot (csrc/trig.h), the sin/cos the rotary kernels use.

trig.h is plain IEEE fp32 arithmetic (fma, rint, mul), so the same source
compiled by g++ with contraction off gives the device's results. It is
checked against float64 sin/cos: |error| <= 1.2e-7 (glibc sinf/cosf reach
3.3e-8; a dropped Taylor term, a wrong Cody-Waite constant or a wrong
quadrant sign shows up as 1e-5 .. 2). Arguments >= 2^20 go to the libm path.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from helpers import ROOT

SRC = r"""
#include "trig.h"
extern "C" void run(const float * x, float * s, float * c, long n) {
    for (long i = 0; i < n; ++i) mi::sincos_rot(x[i], s + i, c + i);
}
"""


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    d = tmp_path_factory.mktemp("trig")
    (d / "t.cpp").write_text(SRC)
    so = d / "libtrig.so"
    subprocess.run(["g++", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-shared", "-fPIC",
                    "-I", os.path.join(ROOT, "hbd-acestep.cpp_amd", "csrc"), str(d / "t.cpp"), "-o", str(so), "-lm"],
                   check=True)
    L = ctypes.CDLL(str(so))
    L.run.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long]
    return L


def _eval(lib, x):
    x = np.ascontiguousarray(x, np.float32)
    s, c = np.empty_like(x), np.empty_like(x)
    lib.run(x.ctypes.data, s.ctypes.data, c.ctypes.data, x.size)
    return s, c


def _err(x, s, c):
    xd = x.astype(np.float64)
    return max(np.max(np.abs(s - np.sin(xd))), np.max(np.abs(c - np.cos(xd))))


def test_sincos_rot_random_range(lib):
    r = np.random.default_rng(0)
    mags = np.concatenate([r.uniform(0, 8, 1_000_000), r.uniform(0, 2 ** 20, 2_000_000),
                           np.exp(r.uniform(np.log(1e-30), np.log(2 ** 20), 1_000_000))]).astype(np.float32)
    x = np.where(r.random(mags.size) < 0.5, -mags, mags).astype(np.float32)
    s, c = _eval(lib, x)
    assert _err(x, s, c) <= 1.2e-7


def test_sincos_rot_quadrant_edges_and_rotary_angles(lib):
    # neighbourhoods of k*pi/4 (reduction and quadrant boundaries)
    k = np.arange(-200_000, 200_000, dtype=np.float64)
    base = (k * np.pi / 4).astype(np.float32)
    x = np.concatenate([np.nextafter(base, np.float32(np.inf)), base, np.nextafter(base, np.float32(-np.inf))])
    s, c = _eval(lib, x)
    assert _err(x, s, c) <= 1.2e-7
    # the rotary angles themselves: fp32 chain pos * ts^i for base 1e4 and 1e6, D = 128
    for fb in (1e4, 1e6):
        ts = np.float32(fb) ** np.float32(-2.0 / 128)
        th = np.arange(0, 40960, dtype=np.float32)
        ang = [th]
        for _ in range(63):
            th = (th * ts).astype(np.float32)
            ang.append(th)
        x = np.concatenate(ang)
        s, c = _eval(lib, x)
        assert _err(x, s, c) <= 1.2e-7


def test_sincos_rot_special_values(lib):
    x = np.array([0.0, -0.0, 1e-45, -1e-45, 2 ** 20 - 0.0625, 2 ** 20, 3e9, np.inf, -np.inf, np.nan], np.float32)
    s, c = _eval(lib, x)
    assert s[0] == 0 and not np.signbit(s[0]) and c[0] == 1
    assert s[1] == 0 and np.signbit(s[1]) and c[1] == 1
    assert s[2] == x[2] and s[3] == x[3]
    assert _err(x[4:7], s[4:7], c[4:7]) <= 1.2e-7  # both sides of the 2^20 switch to libm
    assert np.all(np.isnan(s[7:])) and np.all(np.isnan(c[7:]))
