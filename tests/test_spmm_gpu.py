"""SpMM parity on the GPU: HIP kernels through the C ABI against the oracle
(C restatement of omp_spmm_bf16, block_spmm/inc/bsr_matrix.hpp:954-1000).

Criterion: every output element within 1e-2*sqrt(K_e/32)*max(1,|g|) of the
fp32 golden computed from the same bf16 inputs; every element written (the
output is poisoned with NaN before the launch); the reference's PCC >= 0.99
reported alongside.
"""
import zlib

import numpy as np
import pytest

from helpers import (W, assert_parity, bsr_of, capi, golden_spmm, run_spmm, spmm_k_eff, with_values)

pytestmark = pytest.mark.gpu


def _case(s, b, out_dtype="f32", what=""):
    got = run_spmm(s, b, out_dtype)
    gold = golden_spmm(s, b)
    # A bf16 output is the golden's own T(acc) cast; it is held to the same
    # bound against the fp32 golden (the bound covers the final rounding).
    res = assert_parity(got, gold, spmm_k_eff(s), what)
    return got, gold, res


# --- the reference's single-block known answers (block_spmm/inc/test_suite.hpp:1862-1925)
def test_1_block_id():
    s = W.fill_col(32, 32, 32, 32, 1)
    s.data = W.block_content(1, 32, 32, "ID")
    b = W.dense_content(32, 32, "ID")
    got = run_spmm(s, b)
    np.testing.assert_array_equal(got, np.eye(32, dtype=np.float32))


def test_1_block_uniform():
    s = W.fill_col(32, 32, 32, 32, 1)
    s.data = W.block_content(1, 32, 32, "UNIFORM")
    b = W.dense_content(32, 32, "UNIFORM")
    got = run_spmm(s, b)
    np.testing.assert_array_equal(got, np.full((32, 32), 32.0, np.float32))


def test_1_block_arange():
    s = W.fill_col(32, 32, 32, 32, 1)
    s.data = W.block_content(1, 32, 32, "ARANGE")
    b = W.dense_content(32, 32, "UNIFORM")
    got = run_spmm(s, b)
    a = W.bf16_to_f32(s.data).reshape(32, 32).astype(np.float64)
    expect = np.repeat(a.sum(axis=1, keepdims=True), 32, axis=1)  # integers, exact in fp32
    np.testing.assert_array_equal(got, expect.astype(np.float32))


# --- the small workload (A 1024^2, 10%, N=256), both output types and both entry points
@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_small_workload(out_dtype):
    w = W.workload_spmm_small()
    got, gold, res = _case(w["a"], w["b"], out_dtype, f"small {out_dtype}")
    assert res["pcc"] >= 0.99
    host = capi.host_spmm(capi.Bsr(w["a"].H, w["a"].W, 32, 32, w["a"].indptr, w["a"].indices),
                          w["a"].data, w["b"], out_dtype)
    if out_dtype == "bf16":
        host = W.bf16_to_f32(host)
    np.testing.assert_array_equal(host, got)  # same kernels, same schedule: bit-identical


# --- the density sweep at full size (A 4096^2, B 4096x512)
@pytest.mark.parametrize("density", W.SPMM_SWEEP_DENSITIES)
@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_density_sweep(density, out_dtype):
    w = W.workload_spmm_sweep(density)
    _case(w["a"], w["b"], out_dtype, f"sweep d={density} {out_dtype}")


# --- structures from the reference's generators and hand-written cases
STRUCTS = {
    "fill_row_2x2": lambda: W.fill_row(64, 64, 32, 32, 2),
    "fill_col_4x4": lambda: W.fill_col(128, 128, 32, 32, 6),
    "fill_col_as_reference_dups": lambda: W.fill_col_as_reference(64, 64, 32, 32, 4),
    "diag_1024": lambda: W.fill_diag(1024, 1024, 32, 32, 32),
    "tril_1024": lambda: W.fill_tril(1024, 1024, 32, 32),
    "triu_1024": lambda: W.fill_triu(1024, 1024, 32, 32),
    "multi_diag_1024": lambda: W.fill_multi_diag(1024, 1024, 32, 32, 100),
    # test_big_zero_rows_more (block_spmm/inc/test_suite.hpp:370-398), 64x64 blocks
    "zero_rows_more_R64": lambda: W.BsrArrays(256, 256, 64, 64, np.array([0, 4, 4, 8, 8], np.int32),
                                              np.array([0, 1, 2, 3, 0, 1, 2, 3], np.int32)),
    # test_checkerboard (:554-583)
    "checkerboard_R64": lambda: W.BsrArrays(256, 256, 64, 64, np.array([0, 2, 4, 6, 8], np.int32),
                                            np.array([0, 2, 1, 3, 0, 2, 1, 3], np.int32)),
    # test_random_hang (:584-620): unsorted columns, 64x64 blocks
    "random_hang_R64": lambda: W.BsrArrays(
        1024, 1024, 64, 64,
        np.array([0, 0, 1, 3, 6, 7, 11, 13, 16, 18, 21, 25, 27, 28, 29, 31, 32], np.int32),
        np.array([13, 6, 13, 0, 8, 11, 5, 4, 8, 10, 12, 6, 14, 4, 14, 15, 4, 5, 2, 7, 8, 4, 8, 11, 12,
                  3, 10, 0, 3, 0, 4, 6], np.int32)),
    # test_num_iters_y_2_odd_empty_rows (:646-676)
    "odd_empty_rows_R64": lambda: W.BsrArrays(
        1024, 1024, 64, 64, np.array([0, 1, 1, 1, 2, 2, 3, 3, 3, 6, 7, 7, 7, 7, 7, 7, 8], np.int32),
        np.array([0, 0, 0, 1, 2, 0, 0, 0], np.int32)),
    "tall_blocks_R32_C64": lambda: W.random_positions(256, 256, 32, 64, 4, np.random.default_rng(5)),
    "wide_blocks_R64_C32": lambda: W.random_positions(256, 256, 64, 32, 4, np.random.default_rng(6)),
    "R128_C128": lambda: W.random_positions(1024, 1024, 128, 128, 16, np.random.default_rng(7)),
    "R256_C256_tril": lambda: W.fill_tril(1024, 1024, 256, 256),
    "empty_matrix": lambda: W.BsrArrays(256, 256, 32, 32, np.zeros(9, np.int32), np.zeros(0, np.int32)),
    "last_row_only": lambda: W.BsrArrays(256, 256, 32, 32, np.array([0] * 8 + [1], np.int32),
                                         np.array([7], np.int32)),
}


@pytest.mark.parametrize("name", sorted(STRUCTS))
@pytest.mark.parametrize("N", [32, 64, 256, 512])
def test_structures(name, N):
    s = with_values(STRUCTS[name](), "RAND", seed=zlib.crc32(name.encode()))
    b = W.dense_content(s.W, N, "RAND", np.random.default_rng(N))
    _case(s, b, "f32", f"{name} N={N}")


def test_many_empty_rows_R256():
    """test_many_empty_rows (block_spmm/inc/test_suite.hpp:348-368): 8192x256,
    one 256x256 block in the first row, N=256."""
    s = with_values(W.fill_row(8192, 256, 256, 256, 1), "RAND", seed=3)
    b = W.dense_content(256, 256, "RAND", np.random.default_rng(3))
    got, gold, _ = _case(s, b, "f32", "many_empty_rows")
    assert np.all(got[256:] == 0.0)


# --- skewed rows: the persistent kernel (the plan's choice), the sweep
# kernel, and the per-item kernels with split rows (the reduce kernel adds
# the pieces)
@pytest.mark.parametrize("kernel,split", [("sweep", None), ("persistent", None), ("items", None), ("items", 40)])
def test_skewed_workload_full_size(monkeypatch, kernel, split):
    """The skewed workload as planned (the persistent kernel), on the sweep
    kernel (its shape qualifies for the sweep kernel's automatic choice), on
    the per-item kernels with every row whole, and with the rows over 40
    entries cut into pieces: held to the oracle, and the same bits on a second
    run."""
    if kernel == "items":
        monkeypatch.setenv("BSP_SPMM_STREAM", "0")
    if kernel == "sweep":
        monkeypatch.setenv("BSP_SPMM_SWEEP", "1")
    if split:
        monkeypatch.setenv("BSP_SPMM_SPLIT", str(split))
    w = W.workload_spmm_skewed()
    a = w["a"]
    plan = capi.SpmmPlan(capi.Bsr(a.H, a.W, 32, 32, a.indptr, a.indices), w["N"], "f32")
    info = plan.info()
    assert info["persistent"] == {"sweep": 3, "persistent": 1, "items": 0}[kernel], info
    assert (info["n_split_rows"] > 0) == bool(split)
    if kernel == "sweep":
        # one workgroup per compute unit, 16 units each, one sweep
        assert (info["grid"], info["waves"], info["stages"], info["n_items"]) == (256, 11, 16, 4096), info
    if kernel == "persistent":
        # eight units per workgroup, the longest (101 entries) above a
        # workgroup's share: one workgroup per compute unit, four B loaders,
        # deep rings, two entries per step
        assert (info["grid"], info["waves"], info["stages"], info["a_stages"], info["step_entries"]) == \
            (256, 9, 14, 16, 2), info
    got1 = run_spmm(a, w["b"], "f32", plan=plan)
    got2 = run_spmm(a, w["b"], "f32", plan=plan)
    np.testing.assert_array_equal(got1, got2)  # counters reset, summation order fixed
    assert_parity(got1, golden_spmm(a, w["b"]), spmm_k_eff(a), f"skewed split={split}")
    plan.close()


@pytest.mark.parametrize("split", [1, 3, 7])
def test_forced_splits(monkeypatch, split):
    """Every row cut into pieces of at most `split` entries (per-item kernels)."""
    monkeypatch.setenv("BSP_SPMM_STREAM", "0")
    monkeypatch.setenv("BSP_SPMM_SPLIT", str(split))
    w = W.spmm_workload(1024, 2048, 512, 32, 32, 0.2, seed=11)
    _case(w["a"], w["b"], "f32", f"split={split}")
    _case(w["a"], w["b"], "bf16", f"split={split} bf16")


# Every compiled kernel variant (tile_n, ring depth), on items shorter and
# longer than the ring.
SPMM_VARIANTS = [(128, 4), (128, 6), (128, 8), (256, 3), (256, 4)]


@pytest.mark.parametrize("density", [0.1, 0.5])
@pytest.mark.parametrize("tile_n,stages", SPMM_VARIANTS)
def test_kernel_variants(monkeypatch, tile_n, stages, density):
    monkeypatch.setenv("BSP_SPMM_STREAM", "0")
    monkeypatch.setenv("BSP_SPMM_TILE_N", str(tile_n))
    monkeypatch.setenv("BSP_SPMM_STAGES", str(stages))
    w = W.spmm_workload(2048, 2048, 512, 32, 32, density, seed=12)
    plan = capi.SpmmPlan(capi.Bsr(2048, 2048, 32, 32, w["a"].indptr, w["a"].indices), 512, "f32")
    info = plan.info()
    assert (info["tile_n"], info["stages"]) == (tile_n, stages)
    got = run_spmm(w["a"], w["b"], "f32", plan=plan)
    plan.close()
    assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]),
                  f"variant=({tile_n},{stages}) d={density}")


@pytest.mark.parametrize("N", [32, 96, 160, 288, 384])
def test_partial_last_tile(N):
    """N not a multiple of the tile width: the last tile is partial."""
    w = W.spmm_workload(1024, 1024, N, 32, 32, 0.15, seed=N)
    _case(w["a"], w["b"], "f32", f"N={N}")
    _case(w["a"], w["b"], "bf16", f"N={N} bf16")


def test_linearity_full_size():
    """A*(B1 + B2) == A*B1 + A*B2 within the bound, at the 50% sweep shape.
    B1, B2 hold multiples of 1/64 in [-1/2, 1/2], so B1 + B2 is exact in bf16."""
    w = W.workload_spmm_sweep(0.5)
    a = w["a"]
    rng = np.random.default_rng(21)
    f1 = rng.integers(-32, 33, (4096, 512)).astype(np.float32) / 64
    f2 = rng.integers(-32, 33, (4096, 512)).astype(np.float32) / 64
    b1, b2, b12 = W.bf16_from_f32(f1), W.bf16_from_f32(f2), W.bf16_from_f32(f1 + f2)
    assert np.array_equal(W.bf16_to_f32(b12), f1 + f2)
    s1 = run_spmm(a, b1).astype(np.float64)
    s2 = run_spmm(a, b2).astype(np.float64)
    s12 = run_spmm(a, b12).astype(np.float64)
    assert_parity(s12, s1 + s2, 2 * spmm_k_eff(a), "linearity")


# --- the reference's frozen random patterns (block_spmm/inc/profiling_suite.hpp:95-3507)
def _pattern_names():
    from golden_fixtures import reference_patterns
    return sorted(reference_patterns())


@pytest.mark.parametrize("name", _pattern_names())
def test_reference_frozen_patterns(name):
    """Each frozen structure with seeded random values; N reduced to 64 so the
    oracle stays fast (the structure is what these cases pin)."""
    from golden_fixtures import reference_patterns
    dims, indptr, indices = reference_patterns()[name]
    s = W.BsrArrays(dims["M"], dims["K"], dims["R"], dims["C"], indptr, indices)
    s = with_values(s, "RAND", seed=zlib.crc32(name.encode()))
    b = W.dense_content(s.W, 64, "RAND", np.random.default_rng(7))
    _case(s, b, "f32", name)


def test_small_vectors_fixture():
    from golden_fixtures import small_vectors
    v = small_vectors()
    M, K, R, C = (int(t) for t in v["spmm_shape"])
    s = W.BsrArrays(M, K, R, C, v["spmm_indptr"], v["spmm_indices"], v["spmm_a"])
    assert_parity(run_spmm(s, v["spmm_b"]), v["spmm_golden"], spmm_k_eff(s), "fixture")


def test_bf16_output_rounds_to_nearest_even():
    """bf16 outputs are the fp32 result rounded to nearest, ties to even,
    bit for bit.  C = b1 + b2 + b3 with A = three all-ones blocks in one row
    and bf16 B rows chosen so that the (exact) fp32 sums are ties at bf16
    precision (1 + 2^-8 -> 1, 1 + 3*2^-8 -> 1 + 2^-6, 65280 + 128 -> 65536,
    ...) or just above / below a tie (+-2^-16)."""
    R = C = 32
    N = 32
    a_vals = W.bf16_from_f32(np.ones(3 * R * C, np.float32))
    a = W.BsrArrays(32, 96, R, C, np.array([0, 3], np.int32), np.array([0, 1, 2], np.int32), a_vals)
    cases = [(1.0, 2 ** -8, 0.0), (1.0, 3 * 2 ** -8, 0.0), (1.0, 2 ** -8, 2 ** -16), (-1.0, -2 ** -8, 0.0),
             (256.0, 1.0, 0.0), (2.0 ** -20, 2.0 ** -28, 0.0), (1.0, 2 ** -8, -2 ** -16), (3.0, 2 ** -7, 0.0),
             (0.5, 2 ** -10, 0.0), (1.0, 5 * 2 ** -8, 0.0), (65280.0, 128.0, 0.0), (1.0, -2 ** -9, 0.0)]
    b = np.zeros((96, N), np.float32)
    for j, (x, y, z) in enumerate(cases):
        b[0, j], b[32, j], b[64, j] = x, y, z
    b16 = W.bf16_from_f32(b)
    assert np.array_equal(W.bf16_to_f32(b16), b)  # inputs exactly representable
    gold = golden_spmm(a, b16)  # fp32 sums, exact here
    assert np.array_equal(gold[0, :len(cases)], np.array([x + y + z for x, y, z in cases], np.float32))
    expect = W.bf16_to_f32(W.bf16_from_f32(gold))
    assert list(expect[0, :len(cases)]) == [1.0, 1.015625, 1.0078125, -1.0, 256.0, 2.0 ** -20, 1.0, 3.0,
                                            0.5, 1.015625, 65536.0, 1.0]
    np.testing.assert_array_equal(run_spmm(a, b16, "bf16"), expect)


# ---- row groups: RW stripes of one block row share each B panel -------------

GROUP_VARIANTS = [(2, 6, 64), (4, 4, 128), (4, 5, 128), (8, 3, 256), (8, 4, 256)]


@pytest.mark.parametrize("density", [0.1, 0.5])
@pytest.mark.parametrize("group,stages,R", GROUP_VARIANTS)
def test_row_group_variants(monkeypatch, group, stages, R, density):
    monkeypatch.setenv("BSP_SPMM_GROUP", str(group))
    monkeypatch.setenv("BSP_SPMM_STAGES", str(stages))
    w = W.spmm_workload(2048, 2048, 384, R, R, density, seed=50 + group)
    plan = capi.SpmmPlan(bsr_of(w["a"]), 384, "f32")
    info = plan.info()
    assert (info["group"], info["stages"], info["tile_n"]) == (group, stages, 128)
    got = run_spmm(w["a"], w["b"], "f32", plan=plan)
    plan.close()
    assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]),
                  f"group={group} stages={stages} R={R} d={density}")


@pytest.mark.parametrize("N", [32, 96, 160])
@pytest.mark.parametrize("group", [2, 4, 8])
def test_row_group_partial_tiles_and_bf16(monkeypatch, group, N):
    monkeypatch.setenv("BSP_SPMM_GROUP", str(group))
    R = 32 * group
    w = W.spmm_workload(1024, 1024, N, R, 64, 0.3, seed=60 + N)
    for od in ("f32", "bf16"):
        assert_parity(run_spmm(w["a"], w["b"], od), golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]),
                      f"group={group} N={N} {od}")


@pytest.mark.parametrize("split", [1, 3])
@pytest.mark.parametrize("group", [2, 8])
def test_row_group_split_rows(monkeypatch, group, split):
    monkeypatch.setenv("BSP_SPMM_GROUP", str(group))
    monkeypatch.setenv("BSP_SPMM_SPLIT", str(split))
    R = 32 * group
    w = W.spmm_workload(2048, 2048, 256, R, 32, 0.2, seed=70 + group)
    plan = capi.SpmmPlan(bsr_of(w["a"]), 256, "f32")
    assert plan.info()["group"] == group and plan.info()["n_split_rows"] > 0
    for run in range(2):
        got = run_spmm(w["a"], w["b"], "f32", plan=plan)
        assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]), f"group={group} split={split}")
        if run == 0:
            first = got
    np.testing.assert_array_equal(first, got)  # the split reduction is deterministic
    plan.close()


@pytest.mark.parametrize("R", [256, 128, 64])
def test_row_group_chosen_for_large_blocks(R):
    """The reference's published shape (8192^3 at 25%) with R x R blocks runs
    in groups of R/32 stripes on 256-column tiles without any override;
    checked on a block-row prefix against the oracle (bf16 C for 256, fp32
    for the others)."""
    w = W.workload_spmm_large_blocks(0.25, R=R)
    a = w["a"]
    od = "bf16" if R == 256 else "f32"
    plan = capi.SpmmPlan(bsr_of(a), 8192, od)
    assert plan.info()["group"] == R // 32 and plan.info()["tile_n"] == 256
    got = run_spmm(a, w["b"], od, plan=plan)
    plan.close()
    rows = 1024 if R == 256 else 512
    nb = int(a.indptr[rows // R])
    sub = W.BsrArrays(rows, a.W, R, R, np.ascontiguousarray(a.indptr[:rows // R + 1]),
                      a.indices[:nb], a.data[:nb * R * R])
    assert_parity(got[:rows], golden_spmm(sub, w["b"]), spmm_k_eff(sub), f"8192^3 R={R} prefix")
    # Every row, on a column slice: output column j depends only on column j
    # of B, so the oracle on B's first 64 columns checks all 8192 rows of the
    # default plan (two workgroups per compute unit, reversed second rounds,
    # the row-band map) at a small cost.
    cols = 64
    gold = golden_spmm(a, np.ascontiguousarray(w["b"][:, :cols]))
    assert_parity(got[:, :cols], gold, spmm_k_eff(a), f"8192^3 R={R} all rows, columns 0..{cols - 1}")


@pytest.mark.parametrize("R,C", [(256, 256), (256, 128), (256, 64), (256, 32), (128, 128), (128, 64), (128, 32),
                                 (64, 64), (64, 32)])
@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("split", [0, 3])
@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_row_group_wide_tile(monkeypatch, R, C, waves, split, out_dtype):
    """R x C blocks on the 256-column tile (the wide group kernel over
    R/32 = 8, 4 or 2 stripes), forced on a small shape: C a multiple of 64
    fetches A in entry pairs (C = 64: one pair per block), C = 32 one entry
    at a time (R = 64: 512 bytes per wave with eight waves); with and
    without split rows (whose pieces the reduce kernel adds in the
    256-column layout, and which start at even entries), both outputs, held
    to the oracle, and the same bits on a second run."""
    monkeypatch.setenv("BSP_SPMM_GROUP", str(R // 32))
    monkeypatch.setenv("BSP_SPMM_WIDE_GROUP", "2")
    monkeypatch.setenv("BSP_SPMM_SPLIT", str(split or 100000))
    monkeypatch.setenv("BSP_SPMM_WIDE_WAVES", str(waves))
    w = W.spmm_workload(2048, 2048, 512, R, C, 0.3 if C > 32 else 0.1, seed=90 + split + C + R)
    plan = capi.SpmmPlan(bsr_of(w["a"]), 512, out_dtype)
    info = plan.info()
    assert info["group"] == R // 32 and info["tile_n"] == 256
    assert info["waves"] == (8 if R == 256 else waves)  # four waves of eight stripes would spill
    assert (info["n_split_rows"] > 0) == bool(split)
    got = run_spmm(w["a"], w["b"], out_dtype, plan=plan)
    again = run_spmm(w["a"], w["b"], out_dtype, plan=plan)
    plan.close()
    assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]),
                  f"wide group R={R} C={C} waves={waves} split={split} {out_dtype}")
    np.testing.assert_array_equal(got, again)


@pytest.mark.parametrize("R,stages", [(256, 3), (256, 4), (128, 3), (64, 3)])
@pytest.mark.parametrize("split", [0, 3])
def test_row_group_wide_ring_depths(monkeypatch, R, stages, split):
    """Every compiled (group, ring depth) of the 256-column group kernel,
    forced through BSP_SPMM_STAGES, among them the odd three-stage ring of
    eight-stripe groups (two entry-pair slots), with and without split rows."""
    monkeypatch.setenv("BSP_SPMM_GROUP", str(R // 32))
    monkeypatch.setenv("BSP_SPMM_WIDE_GROUP", "2")
    monkeypatch.setenv("BSP_SPMM_STAGES", str(stages))
    monkeypatch.setenv("BSP_SPMM_SPLIT", str(split or 100000))
    w = W.spmm_workload(2048, 2048, 512, R, R, 0.3, seed=110 + R + stages + split)
    plan = capi.SpmmPlan(bsr_of(w["a"]), 512, "f32")
    info = plan.info()
    assert (info["group"], info["tile_n"], info["stages"]) == (R // 32, 256, stages)
    assert (info["n_split_rows"] > 0) == bool(split)
    got = run_spmm(w["a"], w["b"], "f32", plan=plan)
    plan.close()
    assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]), f"R={R} stages={stages} split={split}")
