"""Writes the committed fixtures under tests/golden/.

1. reference_patterns.npz — the frozen BSR index arrays the reference holds
   as data: the 34 `frozen_parametric_random<M,N,K,R,C,DPPM>` specialisations
   of block_spmm/inc/profiling_suite.hpp:95-3507 and the SDDMM deadlock
   pattern of block_sddmm/inc/test_suite.hpp:114-156.  The arrays are read as
   text from the reference checkout (only the numbers are kept); this script
   is the only thing that reads the reference, and only when it is re-run.
2. small_vectors.npz — small seeded inputs with their fp32 golden outputs
   from the oracle, for regression of the oracle and the kernels.

Run: python tests/golden/make_fixtures.py [/path/to/reference]
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))


def _ints(text: str) -> np.ndarray:
    return np.array([int(t) for t in re.findall(r"-?\d+", text)], dtype=np.int32)


def extract_reference_patterns(ref: Path) -> dict:
    out = {}
    src = (ref / "block_spmm/inc/profiling_suite.hpp").read_text()
    spec = re.compile(
        r"frozen_parametric_random<(\d+),\s*(\d+),\s*(\d+),\s*(\d+),\s*(\d+),\s*(\d+)>\(\)\s*\{"
        r"\s*std::vector<int> indptr = \{(.*?)\};\s*std::vector<int> indices = \{(.*?)\};"
        r"\s*return make_frozen_case\(indptr, indices, (\d+),", re.S)
    for m in spec.finditer(src):
        M, N, K, R, C, dppm = (int(m.group(i)) for i in range(1, 7))
        indptr, indices, nblocks = _ints(m.group(7)), _ints(m.group(8)), int(m.group(9))
        assert indptr.size == M // R + 1 and indptr[-1] == nblocks == indices.size, (M, R, nblocks)
        key = f"spmm_M{M}_N{N}_K{K}_R{R}_C{C}_dppm{dppm}"
        out[key + "__indptr"] = indptr
        out[key + "__indices"] = indices
    src = (ref / "block_sddmm/inc/test_suite.hpp").read_text()
    m = re.search(r"test_deadlock_sweepK_0\(\)\s*\{.*?std::vector<int> indptr = \{(.*?)\};"
                  r"\s*std::vector<int> indices = \{(.*?)\};", src, re.S)
    indptr, indices = _ints(m.group(1)), _ints(m.group(2))
    assert indptr.size == 33 and indptr[-1] == indices.size == 256
    out["sddmm_deadlock_M8192_N8192_K512_R256_C256__indptr"] = indptr
    out["sddmm_deadlock_M8192_N8192_K512_R256_C256__indices"] = indices
    return out


def small_vectors() -> dict:
    import __graft_entry__ as entry
    W = entry.load_package().workloads
    orc = entry._load_oracle()
    out = {}
    rng = np.random.default_rng(20240601)
    # SpMM: 128 x 192 A (32x32 blocks, 40%), B 192 x 64.
    a = W.random_positions(128, 192, 32, 32, 10, rng)
    a.data = W.bf16_from_f32(W.uniform_f32(rng, a.nblocks * 1024))
    b = W.bf16_from_f32(W.uniform_f32(rng, (192, 64)))
    out.update({"spmm_indptr": a.indptr, "spmm_indices": a.indices, "spmm_a": a.data, "spmm_b": b,
                "spmm_shape": np.array([128, 192, 32, 32], np.int32),
                "spmm_golden": orc.spmm(a.indptr, a.indices, a.data, 128, 192, 32, 32, b)})
    # SDDMM: mask 128 x 160 (32x32 blocks, 30%), X 128 x 64, Y 64 x 160, random mask values.
    m = W.random_positions(128, 160, 32, 32, 6, rng)
    m.data = W.bf16_from_f32(W.uniform_f32(rng, m.nblocks * 1024))
    x = W.bf16_from_f32(rng.standard_normal((128, 64), dtype=np.float32))
    y = W.bf16_from_f32(rng.standard_normal((64, 160), dtype=np.float32))
    out.update({"sddmm_indptr": m.indptr, "sddmm_indices": m.indices, "sddmm_mask": m.data,
                "sddmm_x": x, "sddmm_y": y, "sddmm_shape": np.array([128, 160, 32, 32], np.int32),
                "sddmm_golden": orc.sddmm(m.indptr, m.indices, m.data, 128, 160, 32, 32, x, y)})
    return out


def main() -> None:
    ref = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    if ref.exists():
        pats = extract_reference_patterns(ref)
        np.savez_compressed(HERE / "reference_patterns.npz", **pats)
        print(f"reference_patterns.npz: {len(pats) // 2} patterns")
    np.savez_compressed(HERE / "small_vectors.npz", **small_vectors())
    print("small_vectors.npz written")


if __name__ == "__main__":
    main()
