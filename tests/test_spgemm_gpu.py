"""SpGEMM parity on the GPU: the HIP kernel through the C ABI against the
oracle (C restatement of bsr_matrix::spgemm, sparse_common/bsr_matrix.hpp
:741-810).

Structure (indptr, indices) must equal the oracle's bit for bit; values are
held to 1e-2*sqrt(K_e/32)*max(1,|g|) against the fp32 golden, with K_e the
block pairs meeting at the output block times C; every output value is
written (poisoned with NaN first).  At the full workload size the checks are
size-independent closed forms: a block-identity B returns A exactly, all-ones
blocks give pairs * C exactly.
"""
import numpy as np
import pytest

from helpers import (W, assert_parity, bsr_of, capi, golden_spgemm, run_spgemm, spgemm_k_eff,
                     block_pattern)

pytestmark = pytest.mark.gpu


def _rand(H, Wd, R, C, nblocks, seed, content="RAND"):
    rng = np.random.default_rng(seed)
    s = W.random_positions(H, Wd, R, C, nblocks, rng)
    s.data = W.block_content(s.nblocks, R, C, content, rng)
    return s


def _check(a, b, out_dtype="f32", what=""):
    st, got = run_spgemm(a, b, out_dtype)
    ip, ix, gv = golden_spgemm(a, b)
    np.testing.assert_array_equal(st.indptr, ip)
    np.testing.assert_array_equal(st.indices, ix)
    assert got.size == gv.size
    return assert_parity(got, gv, spgemm_k_eff(a, b, st), what)


SHAPES = [(32, 32, 32), (64, 32, 32), (32, 64, 32), (32, 32, 64), (64, 64, 64), (128, 64, 32),
          (32, 96, 64), (256, 32, 32)]


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("R,C,BC", SHAPES)
def test_spgemm_random(R, C, BC, out_dtype):
    a = _rand(8 * R, 10 * C, R, C, 30, R + C)
    b = _rand(10 * C, 8 * BC, C, BC, 30, C + BC)
    _check(a, b, out_dtype, f"R={R} C={C} BC={BC} {out_dtype}")


@pytest.mark.parametrize("C", [32, 64])
def test_spgemm_long_product_lists(C):
    """A dense block row times a dense block column: 4096 / C pairs per
    output block, C / 32 products each (well past the ring depth)."""
    a = W.fill_row(64, 4096, 32, C, 2 * (4096 // C))
    b = W.fill_row(4096, 64, C, 32, 2 * (4096 // C))
    rng = np.random.default_rng(C)
    a.data = W.block_content(a.nblocks, 32, C, "RAND", rng)
    b.data = W.block_content(b.nblocks, C, 32, "RAND", rng)
    _check(a, b, "f32", f"long C={C}")


def test_spgemm_duplicates_and_empty_rows():
    """A duplicate A block contributes once per stored copy; empty block rows
    of A and empty block rows of B leave no output."""
    rng = np.random.default_rng(11)
    a = W.BsrArrays(256, 128, 32, 32, np.array([0, 3, 3, 4, 6, 6, 7, 7, 8], np.int32),
                    np.array([2, 0, 2, 1, 1, 3, 0, 3], np.int32))
    a.data = W.block_content(a.nblocks, 32, 32, "RAND", rng)
    b = W.BsrArrays(128, 128, 32, 32, np.array([0, 2, 2, 3, 5], np.int32), np.array([0, 3, 1, 0, 2], np.int32))
    b.data = W.block_content(b.nblocks, 32, 32, "RAND", rng)
    _check(a, b, "f32", "duplicates")
    _check(a, b, "bf16", "duplicates bf16")


def test_spgemm_single_output_block_and_empty_product():
    a = _rand(32, 64, 32, 32, 2, 3)
    b = W.fill_row(64, 32, 32, 32, 2)
    b.data = W.block_content(2, 32, 32, "RAND", np.random.default_rng(4))
    _check(a, b, "f32", "one block")
    # A's columns meet only B's empty rows: no output blocks, nothing launched.
    a2 = W.BsrArrays(64, 128, 32, 32, np.array([0, 1, 2], np.int32), np.array([0, 1], np.int32))
    a2.data = W.block_content(2, 32, 32, "RAND", np.random.default_rng(5))
    b2 = W.BsrArrays(128, 64, 32, 32, np.array([0, 0, 0, 1, 2], np.int32), np.array([0, 1], np.int32))
    b2.data = W.block_content(2, 32, 32, "RAND", np.random.default_rng(6))
    st, got = run_spgemm(a2, b2)
    assert st.nblocks == 0 and got.size == 0
    assert np.array_equal(st.indptr, [0, 0, 0])


def test_spgemm_workload_against_oracle():
    """The workload's density at 4096 x 4096 (oracle in seconds)."""
    w = W.workload_spgemm(n=4096, density=0.10, seed=W.SEED_BASE + 7)
    res = _check(w["a"], w["b"], "f32", "4096 10%")
    assert res["pcc"] > 0.9999


def test_spgemm_plan_reuse_structure_and_host_entry():
    a = _rand(512, 512, 64, 32, 40, 21)
    b = _rand(512, 512, 32, 64, 40, 22)
    plan = capi.SpgemmPlan(bsr_of(a), bsr_of(b), "f32")
    sym = capi.spgemm_symbolic(bsr_of(a), bsr_of(b))
    np.testing.assert_array_equal(plan.structure.indptr, sym.indptr)
    np.testing.assert_array_equal(plan.structure.indices, sym.indices)
    info = plan.info()
    assert info["kind"] == 4 and info["n_items"] == sym.nblocks * 2 * 2
    _, v1 = run_spgemm(a, b, plan=plan)
    _, v2 = run_spgemm(a, b, plan=plan)
    np.testing.assert_array_equal(v1, v2)  # deterministic
    hst, hv = capi.host_spgemm(bsr_of(a), a.data, bsr_of(b), b.data, "f32")
    np.testing.assert_array_equal(hst.indices, sym.indices)
    np.testing.assert_array_equal(hv, v1)
    plan.close()


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_spgemm_full_size_block_identity(out_dtype):
    """A (the benchmark's 8192 x 8192, 5%) times the block-identity: C = A,
    exactly (one nonzero term per value)."""
    w = W.workload_spgemm()
    a = w["a"]
    b = W.fill_diag(a.W, a.W, 32, 32, a.W // 32)
    b.data = W.block_content(b.nblocks, 32, 32, "ID")
    st, got = run_spgemm(a, b, out_dtype)
    np.testing.assert_array_equal(st.indptr, a.indptr)
    np.testing.assert_array_equal(st.indices, a.indices)
    np.testing.assert_array_equal(got, W.bf16_to_f32(a.data))


def test_spgemm_full_size_all_ones():
    """The benchmark's structures with all-ones blocks: every output value is
    (pairs at its block) * 32, exact in fp32."""
    w = W.workload_spgemm()
    a, b = w["a"], w["b"]
    a = W.BsrArrays(a.H, a.W, 32, 32, a.indptr, a.indices, W.block_content(a.nblocks, 32, 32, "UNIFORM"))
    b = W.BsrArrays(b.H, b.W, 32, 32, b.indptr, b.indices, W.block_content(b.nblocks, 32, 32, "UNIFORM"))
    st, got = run_spgemm(a, b)
    pairs = block_pattern(a) @ block_pattern(b)
    assert st.nblocks == int((pairs > 0).sum())
    rows = np.repeat(np.arange(st.nbrows), np.diff(st.indptr))
    np.testing.assert_array_equal(got, np.repeat(pairs[rows, st.indices] * 32.0, 1024).astype(np.float32))
