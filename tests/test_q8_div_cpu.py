"""Host check of the Q8_0 scale division used by the quantize kernels.

The kernels compute d = amax / 127 as q0 = amax * RN(1/127) corrected by one
fma (r = fma(-q0, 127, amax); d = fma(r, RN(1/127), q0)). This test runs that
sequence and the IEEE division over every non-negative finite float (2^31
values, with denormals, which the kernels preserve) and requires identical
bits: a single mismatching amax would change a stored fp16 scale.
"""
import os
import subprocess

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
int main(void) {
    const float c = 1.0f / 127.0f;
    long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t b = 0; b < 0x7f800000LL; ++b) {
        uint32_t u = (uint32_t) b, a1, a2;
        float    x, ref, q;
        memcpy(&x, &u, 4);
        ref = x / 127.0f;
        const float q0 = x * c;
        q = fmaf(fmaf(-q0, 127.0f, x), c, q0);
        memcpy(&a1, &ref, 4);
        memcpy(&a2, &q, 4);
        bad += a1 != a2;
    }
    printf("%ld\n", bad);
    return 0;
}
"""


def test_div127_fma_sequence_is_exact_for_all_floats(tmp_path):
    (tmp_path / "d.c").write_text(SRC)
    exe = tmp_path / "d"
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", str(tmp_path / "d.c"),
                    "-o", str(exe), "-lm"], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(max(1, min(os.cpu_count() or 1, 16))))
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600, check=True)
    assert out.stdout.strip() == "0"
