"""Writes tests/golden/rock4_reference.npz: the ROCK4 coefficient tables the
reference's STORK4 solver reads (src/solvers/solver-stork4-constants.h:14-1273:
the 50 tabulated degrees STORK4_MS, the finishing coefficients STORK4_FPA
[50][6] and STORK4_FPB [50][4], and the 4382 recurrence coefficients
STORK4_RECF). They are Abdulle's published ROCK4 constants (SIAM J. Sci.
Comput. 2002), caller data of mi_stork4_step, kept here as a fixture so the
GPU tests can run the step with the reference's own tables (the reference
tree is not present where the GPU tests run).

Each array is read by name from the header's initializer text and checked
for its declared length; nothing else of the header is used.

Run from the repository root (needs the reference checkout):
    python tests/golden/make_rock4_tables.py
"""
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/src/solvers/solver-stork4-constants.h"
NUM = r"[-+]?(?:\d+\.\d*|\.\d+|\d+)(?:[eE][-+]?\d+)?"


def _array(text: str, name: str, count: int, dtype) -> np.ndarray:
    """The numbers of `static const <type> name[...] = { ... };`, in order."""
    m = re.search(r"\b" + name + r"\s*(?:\[\d+\])+\s*=\s*\{(.*?)\}\s*;", text, flags=re.S)
    if m is None:
        raise ValueError(f"{name} not found in {SRC}")
    vals = re.findall(NUM, m.group(1))
    if len(vals) != count:
        raise ValueError(f"{name}: {len(vals)} values, expected {count}")
    return np.array([float(v) for v in vals]).astype(dtype)


def main():
    text = open(SRC).read()
    ms = _array(text, "STORK4_MS", 50, np.int32)
    fpa = _array(text, "STORK4_FPA", 50 * 6, np.float64).reshape(50, 6)
    fpb = _array(text, "STORK4_FPB", 50 * 4, np.float64).reshape(50, 4)
    recf = _array(text, "STORK4_RECF", 4382, np.float64)
    if int(np.sum(2 * ms.astype(np.int64) - 1)) != recf.size:
        raise ValueError("recurrence blocks (2m - 1 per degree) do not add up to STORK4_RECF's length")
    out = os.path.join(HERE, "rock4_reference.npz")
    np.savez_compressed(out, ms=ms, fpa=fpa, fpb=fpb, recf=recf)
    print(f"wrote {out}: {ms.size} degrees ({ms[0]}..{ms[-1]}), recf {recf.size}")


if __name__ == "__main__":
    main()
