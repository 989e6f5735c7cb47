"""The persistent SpMM kernel (spmm_stream_kernel) on the GPU against the
oracle (omp_spmm_bf16, block_spmm/inc/bsr_matrix.hpp:954-1000): every compiled
variant and workgroups-per-compute-unit setting, streams that cross many
units (empty stripes among them), streams longer than the word prefetch, and
grids with more workgroups than units.  Outputs are poisoned with NaN before
each launch, so an unwritten element fails."""
import numpy as np
import pytest

from helpers import W, assert_parity, bsr_of, capi, golden_spmm, run_spmm, spmm_k_eff, strided_run, with_values

pytestmark = pytest.mark.gpu

# (tile, B ring, A ring, B loader waves, pipelines per workgroup, entries per
# ring step, stripes per unit) of BSP_SPMM_STREAM_VARIANTS in csrc/bsp_kernels.hpp
STREAM_VARIANTS = [(128, 8, 8, 2, 1, 2, 1), (128, 14, 16, 4, 1, 2, 1), (128, 8, 8, 2, 1, 2, 2),
                   (128, 6, 12, 2, 1, 2, 1), (128, 6, 12, 2, 1, 1, 1), (128, 6, 12, 4, 1, 1, 1),
                   (128, 4, 16, 4, 1, 1, 1), (128, 8, 16, 8, 1, 1, 1), (256, 4, 16, 4, 1, 1, 1),
                   (256, 5, 16, 8, 1, 1, 1), (256, 6, 8, 8, 1, 1, 1), (128, 6, 12, 2, 2, 1, 1),
                   (128, 5, 12, 2, 2, 1, 1)]
DEFAULT = (128, 8, 8, 2, 1, 2, 1)   # uniform rows
SKEWED = (128, 14, 16, 4, 1, 2, 1)  # skewed rows: one workgroup per compute unit
PAIRS = (128, 8, 8, 2, 1, 2, 2)     # stripe pairs that share most block columns


def _lds(v):
    pairs_words = 8 * v[2] if v[6] > 1 else 0
    return v[4] * (64 * v[0] * v[1] + 2048 * v[2] * v[6] + pairs_words) + (16384 * v[0] // 128 if v[4] > 1 else 0)


def _waves(v):
    return (4 * v[6] + 1 + v[3]) * v[4]


def _stream_env(monkeypatch, v, wpc=None):
    monkeypatch.setenv("BSP_SPMM_STREAM", "1")
    monkeypatch.setenv("BSP_SPMM_STREAM_VARIANT", ",".join(map(str, v)))
    monkeypatch.setenv("BSP_SPMM_PAIRS", "2" if v[6] > 1 else "0")
    if wpc:
        monkeypatch.setenv("BSP_SPMM_STREAM_WPC", str(wpc))


def _check(a, b, out_dtype, what, v=None, wpc=None):
    plan = capi.SpmmPlan(bsr_of(a), b.shape[1], out_dtype)
    info = plan.info()
    assert info["persistent"] >= 1, f"{what}: plan is not persistent ({info})"
    if v is not None:
        assert (info["tile_n"], info["stages"], info["a_stages"], info["waves"], info["persistent"],
                info["step_entries"], info["stripes_per_unit"]) == (v[0], v[1], v[2], _waves(v), v[4], v[5], v[6])
    if wpc is not None:
        assert info["grid"] == 256 * wpc
    got = run_spmm(a, b, out_dtype, plan=plan)
    got2 = run_spmm(a, b, out_dtype, plan=plan)
    plan.close()
    np.testing.assert_array_equal(got, got2, err_msg=f"{what}: two runs differ")
    assert_parity(got, golden_spmm(a, b), spmm_k_eff(a), what)
    return got


@pytest.mark.parametrize("density", [0.1, 0.5])
@pytest.mark.parametrize("v", STREAM_VARIANTS)
def test_stream_variants(monkeypatch, v, density):
    """Every variant, with as many workgroups per compute unit as its LDS
    allows (one or two), both output types."""
    for wpc in (1, 2):
        if wpc * _lds(v) > 160 * 1024 or (v[4] > 1 and wpc > 1):
            continue
        _stream_env(monkeypatch, v, wpc)
        w = W.spmm_workload(2048, 2048, 512, 32, 32, density, seed=80 + wpc)
        for od in ("f32", "bf16"):
            _check(w["a"], w["b"], od, f"variant={v} wpc={wpc} d={density} {od}", v, wpc)


@pytest.mark.parametrize("v", [DEFAULT, SKEWED, PAIRS, (128, 6, 12, 2, 1, 1, 1), (256, 4, 16, 4, 1, 1, 1), (128, 6, 12, 2, 2, 1, 1)])
def test_stream_many_units_per_workgroup(monkeypatch, v):
    """32768 rows x 1024 columns at 0.2%: 8192 or 4096 units on 256-512
    workgroups (16 per workgroup), many of them empty stripes, stored as zeros."""
    _stream_env(monkeypatch, v)
    w = W.spmm_workload(32768, 4096, 1024, 32, 32, 0.002, seed=91)
    a = w["a"]
    assert (np.diff(a.indptr) == 0).sum() > 100  # empty stripes among the units
    _check(a, w["b"], "f32", f"many units {v}")


@pytest.mark.parametrize("v", [DEFAULT, SKEWED, PAIRS, (128, 6, 12, 2, 1, 1, 1), (256, 5, 16, 8, 1, 1, 1), (128, 6, 12, 2, 2, 1, 1)])
def test_stream_long_rows(monkeypatch, v):
    """A few rows of 200-400 entries (streams far longer than the ring and the
    word prefetch) among short ones."""
    _stream_env(monkeypatch, v)
    rng = np.random.default_rng(92)
    nbr, nbc = 64, 512
    counts = rng.integers(0, 6, nbr)
    counts[[3, 17, 40]] = [400, 250, 200]
    indices = np.concatenate([np.sort(rng.choice(nbc, c, replace=False)) for c in counts]).astype(np.int32)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    a = W.BsrArrays(nbr * 32, nbc * 32, 32, 32, indptr, indices)
    a.data = W.block_content(a.nblocks, 32, 32, "RAND", rng)
    b = W.dense_content(nbc * 32, 256, "RAND", rng)
    _check(a, b, "f32", f"long rows {v}")
    _check(a, b, "bf16", f"long rows {v} bf16")


@pytest.mark.parametrize("v", [DEFAULT, PAIRS, (128, 6, 12, 2, 1, 1, 1)])
def test_stream_fewer_units_than_workgroups(monkeypatch, v):
    """A 64x128 problem: 2 units for 512 workgroups; the rest stream nothing."""
    _stream_env(monkeypatch, v, 2)
    w = W.spmm_workload(64, 256, 128, 32, 32, 0.5, seed=93)
    _check(w["a"], w["b"], "f32", "2 units")


@pytest.mark.parametrize("v", [DEFAULT, SKEWED, PAIRS, (128, 6, 12, 2, 1, 2, 1), (128, 6, 12, 2, 1, 1, 1)])
def test_stream_step_tails(monkeypatch, v):
    """One unit per workgroup with every stream length from 0 to 40 entries:
    with two entries per step, odd and even lengths end differently, and
    lengths below the ring depth never reach the steady state."""
    _stream_env(monkeypatch, v)
    rng = np.random.default_rng(97)
    counts = np.arange(41)
    rng.shuffle(counts)
    nbc = 64
    indices = np.concatenate([np.sort(rng.choice(nbc, c, replace=False)) for c in counts]).astype(np.int32)
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    a = W.BsrArrays(len(counts) * 32, nbc * 32, 32, 32, indptr, indices)
    a.data = W.block_content(a.nblocks, 32, 32, "RAND", rng)
    b = W.dense_content(nbc * 32, 128, "RAND", rng)
    plan = capi.SpmmPlan(bsr_of(a), 128, "f32")
    info = plan.info()
    plan.close()
    units = (len(counts) + 1) // 2 if v[6] > 1 else len(counts)
    assert info["n_items"] == units and info["grid"] >= units  # one unit per workgroup
    _check(a, b, "f32", f"tails {v}")
    _check(a, b, "bf16", f"tails {v} bf16")


@pytest.mark.parametrize("v", [DEFAULT, PAIRS, (128, 6, 12, 2, 2, 1, 1)])
def test_stream_empty_matrix(monkeypatch, v):
    """No stored blocks: every unit is an empty stripe, every tile stored as zeros."""
    pipes = v[4]
    _stream_env(monkeypatch, v)
    a = W.BsrArrays(1024, 1024, 32, 32, np.zeros(33, np.int32), np.zeros(0, np.int32))
    a.data = np.zeros(0, np.uint16)
    b = W.dense_content(1024, 256, "RAND", np.random.default_rng(94))
    plan = capi.SpmmPlan(bsr_of(a), 256, "f32")
    assert plan.info()["persistent"] == pipes
    got = run_spmm(a, b, "f32", plan=plan)
    plan.close()
    assert np.all(got == 0.0)


@pytest.mark.parametrize("v", [DEFAULT, (128, 6, 12, 2, 2, 1, 1)])
@pytest.mark.parametrize("R,C", [(64, 64), (32, 96), (96, 32)])
def test_stream_other_block_shapes(monkeypatch, R, C, v):
    """Blocks other than 32x32 cut into 32-row stripes (no row groups)."""
    monkeypatch.setenv("BSP_SPMM_GROUP", "1")
    _stream_env(monkeypatch, v)
    w = W.spmm_workload(1536, 1536, 256, R, C, 0.2, seed=95 + R + C)
    _check(w["a"], w["b"], "f32", f"R={R} C={C}")


@pytest.mark.parametrize("density", W.SPMM_SWEEP_DENSITIES)
def test_default_plan_variant(density):
    """The density sweep's plans take the default variant, two workgroups per
    compute unit (what the sweep tests and the bench run)."""
    w = W.workload_spmm_sweep(density)
    a = w["a"]
    plan = capi.SpmmPlan(bsr_of(a), w["b"].shape[1], "f32")
    info = plan.info()
    plan.close()
    v = DEFAULT
    assert (info["persistent"], info["tile_n"], info["stages"], info["a_stages"], info["waves"],
            info["step_entries"], info["stripes_per_unit"], info["grid"]) == \
        (1, v[0], v[1], v[2], _waves(v), v[5], v[6], 512), info


def _pair_structures():
    """Block-row structures for the stripe-pair tests (128 stripes of 32x32
    blocks over 128 block columns unless noted; the 4096^2 25% sweep
    workload)."""
    rng = np.random.default_rng(98)
    nbc = 128

    def mk(rows, nbc=nbc):
        indices = np.concatenate([np.asarray(r, np.int32) for r in rows]) if rows else np.zeros(0, np.int32)
        indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
        a = W.BsrArrays(len(rows) * 32, nbc * 32, 32, 32, indptr, indices)
        a.data = W.block_content(a.nblocks, 32, 32, "RAND", rng)
        return a

    base = [np.sort(rng.choice(nbc, int(rng.integers(20, 60)), replace=False)) for _ in range(64)]
    near = []
    for r in base:  # each pair: the same columns, one of them moved
        r2 = r.copy()
        free = np.setdiff1d(np.arange(nbc), r)
        r2[0] = free[0]
        near += [r, np.sort(r2)]
    band = [np.arange(min(max(i - 8, 0), nbc - 16), min(max(i - 8, 0), nbc - 16) + 16) for i in range(128)]
    equal = [np.sort(rng.choice(nbc, 48, replace=False)) for _ in range(64)]
    return {
        "banded, 16 blocks a row": mk(band),
        "identical pairs": mk([r for r in base for _ in range(2)]),
        "identical pairs, 48 blocks a row": mk([r for r in equal for _ in range(2)]),
        "near-identical pairs": mk(near),
        "uniform 25%": W.workload_spmm_sweep(0.25)["a"],
        "every second stripe empty": mk([x for r in base for x in (r, [])]),
        "odd stripe count": mk([r for r in base for _ in range(2)][:-1]),
    }


@pytest.mark.parametrize("name", ["banded, 16 blocks a row", "identical pairs", "identical pairs, 48 blocks a row",
                                  "near-identical pairs", "uniform 25%", "every second stripe empty",
                                  "odd stripe count"])
def test_stripe_pairs_bitwise_equal_to_one_stripe(monkeypatch, name):
    """Stripe pairs keep each stripe's own summation order (its blocks in CSR
    order), so their output is the single-stripe kernel's bit for bit, and
    both are held to the oracle."""
    a = _pair_structures()[name]
    b = W.dense_content(a.W, 512, "RAND", np.random.default_rng(99))
    for od in ("f32", "bf16"):
        outs = {}
        for mode in ("0", "2"):
            monkeypatch.setenv("BSP_SPMM_PAIRS", mode)
            plan = capi.SpmmPlan(bsr_of(a), 512, od)
            info = plan.info()
            assert info["persistent"] == 1 and info["stripes_per_unit"] == (2 if mode == "2" else 1), info
            plan.close()
            outs[mode] = _check(a, b, od, f"{name} pairs={mode} {od}")
        np.testing.assert_array_equal(outs["0"], outs["2"], err_msg=f"{name} {od}: pairs differ from one stripe")


def test_stripe_pairs_chosen_only_where_they_stream_less():
    """The plan takes stripe pairs where its estimate of the bytes each
    compute unit streams comes out lower for them: banded rows, identical
    pairs of equal rows.  It keeps one stripe per unit on uniform-random rows
    and on identical pairs of rows of 20-60 blocks, where the largest pair
    (59 entries of 12 KB, 850 KB with the one-workgroup factor) streams more
    than a compute unit's share of single stripes (74 entries of 10 KB)."""
    s = _pair_structures()
    for name, want in (("banded, 16 blocks a row", 2), ("identical pairs, 48 blocks a row", 2),
                       ("identical pairs", 1), ("near-identical pairs", 1), ("uniform 25%", 1)):
        a = s[name]
        plan = capi.SpmmPlan(bsr_of(a), 512, "f32")
        info = plan.info()
        plan.close()
        assert info["stripes_per_unit"] == want, (name, info)
        if want == 2:
            assert (info["stages"], info["a_stages"], info["waves"], info["grid"]) == \
                (PAIRS[1], PAIRS[2], _waves(PAIRS), 256), info


@pytest.mark.parametrize("density", [0.25, 0.5])
def test_units_rotated_or_in_csr_order(monkeypatch, density):
    """The plan rotates each persistent unit to start at its column group's
    share of the block columns (two column groups at 4096^2 x 512); with
    BSP_SPMM_ROTATE=0 the units run in CSR order.  Both orders are held to
    the oracle and repeat bit for bit; they differ only in the fp32
    summation order of a unit."""
    w = W.workload_spmm_sweep(density)
    outs = {}
    for rot in ("1", "0"):
        monkeypatch.setenv("BSP_SPMM_ROTATE", rot)
        plan = capi.SpmmPlan(bsr_of(w["a"]), 512, "f32")
        assert plan.info()["units_rotated"] == int(rot), plan.info()
        plan.close()
        outs[rot] = _check(w["a"], w["b"], "f32", f"{density} rotate={rot}")  # oracle + repeat
    assert not np.array_equal(outs["1"], outs["0"]), "the rotation changed no unit's order"


def _unsorted_with_duplicates(seed):
    """4096^2 in 32x32 blocks, about 18% of the positions: every row's columns
    shuffled and one column in five repeated (the reference's FILL_COL yields
    such rows), so a rotation point falls inside unsorted runs."""
    rng = np.random.default_rng(seed)
    base = W.random_positions(4096, 4096, 32, 32, 3000, rng)
    ptr, idx = [0], []
    for i in range(base.nbrows):
        cols = list(base.indices[base.indptr[i]:base.indptr[i + 1]])
        cols += [c for c in cols if rng.random() < 0.2]
        rng.shuffle(cols)
        idx += cols
        ptr.append(len(idx))
    return W.BsrArrays(4096, 4096, 32, 32, np.array(ptr, np.int32), np.array(idx, np.int32))


@pytest.mark.parametrize("name", ["R32_C64", "R32_C128", "unsorted_duplicates"])
def test_rotated_units_multi_entry_blocks_and_unsorted_rows(monkeypatch, name):
    """Rotation with two column groups (4096^2 x 512) where a block is several
    32-column entries (C = 64, 128: the rotation starts at a block boundary)
    and where rows hold unsorted and repeated columns; held to the oracle in
    both orders."""
    rng = np.random.default_rng(41)
    a = {"R32_C64": lambda: W.random_positions(4096, 4096, 32, 64, 1500, rng),
         "R32_C128": lambda: W.random_positions(4096, 4096, 32, 128, 700, rng),
         "unsorted_duplicates": lambda: _unsorted_with_duplicates(43)}[name]()
    a = with_values(a, "RAND", seed=44)
    b = W.dense_content(a.W, 512, "RAND", np.random.default_rng(45))
    for rot in ("1", "0"):
        monkeypatch.setenv("BSP_SPMM_ROTATE", rot)
        _check(a, b, "f32", f"{name} rotate={rot}")



@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("v", [DEFAULT, PAIRS, (128, 6, 12, 2, 2, 1, 1)])
def test_strided_b_and_c(monkeypatch, v, out_dtype):
    """B and C as column slices of wider tensors (ldb = N + 64, ldc = N + 128)
    with NaN-poisoned padding: the result equals the contiguous run bit for
    bit, is held to the oracle, and the padding columns stay untouched."""
    import torch
    _stream_env(monkeypatch, v)
    w = W.spmm_workload(2048, 2048, 512, 32, 32, 0.1, seed=91)
    a, b = w["a"], w["b"]
    N = b.shape[1]
    plan = capi.SpmmPlan(bsr_of(a), N, out_dtype)
    assert plan.info()["persistent"] >= 1
    ref = run_spmm(a, b, out_dtype, plan=plan)

    def call(da, bv, cv):
        plan.run(da, bv, cv, stream=torch.cuda.current_stream().cuda_stream)
    got, pad, pad0 = strided_run(a, b, out_dtype, N + 64, N + 128, call)
    plan.close()
    np.testing.assert_array_equal(got, ref, err_msg=f"strided {v} {out_dtype}")
    np.testing.assert_array_equal(pad.view(np.uint8), pad0.view(np.uint8), err_msg="padding of C was written")
    assert_parity(got, golden_spmm(a, b), spmm_k_eff(a), f"strided {v} {out_dtype}")
