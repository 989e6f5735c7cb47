"""Loaders for the committed fixtures in tests/golden/ (made by
tests/golden/make_fixtures.py)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def reference_patterns() -> dict:
    """{name: (shape dict, indptr, indices)} for the reference's frozen SpMM
    patterns (block_spmm/inc/profiling_suite.hpp:95-3507)."""
    z = np.load(GOLDEN / "reference_patterns.npz", allow_pickle=False)
    out = {}
    for k in z.files:
        name, part = k.split("__")
        if not name.startswith("spmm_") or part != "indptr":
            continue
        dims = dict((m[0], int(m[1:])) for m in name.split("_")[1:] if m[0] in "MNKRC" and m[1:].isdigit())
        out[name] = (dims, z[name + "__indptr"], z[name + "__indices"])
    return out


def sddmm_deadlock_pattern():
    """indptr, indices of test_deadlock_sweepK_0 (block_sddmm/inc/test_suite.hpp:114-156)."""
    z = np.load(GOLDEN / "reference_patterns.npz", allow_pickle=False)
    key = "sddmm_deadlock_M8192_N8192_K512_R256_C256"
    return z[key + "__indptr"], z[key + "__indices"]


def small_vectors() -> dict:
    z = np.load(GOLDEN / "small_vectors.npz", allow_pickle=False)
    return {k: z[k] for k in z.files}
