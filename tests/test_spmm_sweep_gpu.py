"""The sweep SpMM kernel (spmm_sweep_kernel: one workgroup per compute unit
holding up to 16 stripe x 128-column units, entries merged by block column)
on the GPU against the oracle (omp_spmm_bf16,
block_spmm/inc/bsr_matrix.hpp:954-1000).  Outputs are poisoned with NaN
before each launch, so an unwritten element fails; every case also runs
twice and must give the same bits."""
import numpy as np
import pytest

from helpers import W, assert_parity, bsr_of, capi, golden_spmm, run_spmm, spmm_k_eff, strided_run, with_values

pytestmark = pytest.mark.gpu


def _check(a, b, out_dtype, what, expect_sweeps=None):
    plan = capi.SpmmPlan(bsr_of(a), b.shape[1], out_dtype)
    info = plan.info()
    assert info["persistent"] == 3, f"{what}: plan is not the sweep kernel ({info})"
    got = run_spmm(a, b, out_dtype, plan=plan)
    got2 = run_spmm(a, b, out_dtype, plan=plan)
    plan.close()
    np.testing.assert_array_equal(got, got2, err_msg=f"{what}: two runs differ")
    assert_parity(got, golden_spmm(a, b), spmm_k_eff(a), what)
    return got


@pytest.fixture
def sweep(monkeypatch):
    monkeypatch.setenv("BSP_SPMM_SWEEP", "2")
    return monkeypatch


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_sweep_skewed_workload(monkeypatch, out_dtype):
    """The skewed 16384^2 x 1024 workload qualifies for the sweep kernel's
    automatic choice (BSP_SPMM_SWEEP=1)."""
    monkeypatch.setenv("BSP_SPMM_SWEEP", "1")
    w = W.workload_spmm_skewed()
    _check(w["a"], w["b"], out_dtype, f"skewed {out_dtype}")


@pytest.mark.parametrize("cg", ["1", "2", "4", "8"])
def test_sweep_column_groups(sweep, cg):
    sweep.setenv("BSP_SPMM_XCD_COLS", cg)
    w = W.spmm_workload(4096, 4096, 1024, 32, 32, 0.05, seed=71)
    _check(w["a"], w["b"], "f32", f"column groups {cg}")


def test_sweep_two_sweeps_per_workgroup(sweep):
    """16384 x 8192 with N = 2048: 8192 units, two sweeps per workgroup (the
    first sweep's stores sit in the load queue in front of the second's
    loads)."""
    w = W.spmm_workload(16384, 8192, 2048, 32, 32, 0.01, seed=72)
    plan = capi.SpmmPlan(bsr_of(w["a"]), 2048, "f32")
    assert plan.info()["n_items"] == 8192
    plan.close()
    _check(w["a"], w["b"], "f32", "two sweeps")


@pytest.mark.parametrize("density", [0.002, 0.2])
def test_sweep_low_and_high_density(sweep, density):
    """Few entries (most sweeps short, odd counts padded) and many."""
    w = W.spmm_workload(4096, 4096, 512, 32, 32, density, seed=73)
    for od in ("f32", "bf16"):
        _check(w["a"], w["b"], od, f"density {density} {od}")


@pytest.mark.parametrize("R,C", [(64, 64), (32, 128), (128, 32), (256, 256)])
def test_sweep_larger_blocks(sweep, R, C):
    w = W.spmm_workload(2048, 2048, 512, R, C, 0.1, seed=74 + R + C)
    _check(w["a"], w["b"], "f32", f"R={R} C={C}")


def test_sweep_empty_rows_duplicates_and_empty_matrix(sweep):
    """Rows with shuffled and repeated block columns and a third of the rows
    empty; then a matrix with no blocks at all (every tile stored as zeros)."""
    rng = np.random.default_rng(75)
    ptr, idx = [0], []
    for i in range(128):
        cols = [] if rng.random() < 0.33 else list(rng.choice(128, size=int(rng.integers(1, 14)), replace=False))
        cols += [c for c in cols if rng.random() < 0.25]
        rng.shuffle(cols)
        idx += cols
        ptr.append(len(idx))
    a = with_values(W.BsrArrays(4096, 4096, 32, 32, np.array(ptr, np.int32), np.array(idx, np.int32)), "RAND", 76)
    b = W.dense_content(4096, 512, "RAND", np.random.default_rng(77))
    _check(a, b, "f32", "empty rows and duplicates")
    e = W.BsrArrays(4096, 4096, 32, 32, np.zeros(129, np.int32), np.zeros(0, np.int32))
    e.data = np.zeros(16, np.uint16)
    plan = capi.SpmmPlan(bsr_of(e), 512, "f32")
    assert plan.info()["persistent"] == 3
    got = run_spmm(e, b, "f32", plan=plan)
    plan.close()
    assert np.all(got == 0.0)


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_sweep_strided_b_and_c(sweep, out_dtype):
    """B and C as column slices of wider tensors (ldb = N + 64, ldc = N + 128)
    with NaN-poisoned padding: equal to the contiguous run, padding intact."""
    import torch
    w = W.spmm_workload(4096, 4096, 512, 32, 32, 0.05, seed=78)
    a, b = w["a"], w["b"]
    N = b.shape[1]
    plan = capi.SpmmPlan(bsr_of(a), N, out_dtype)
    assert plan.info()["persistent"] == 3
    ref = run_spmm(a, b, out_dtype, plan=plan)

    def call(da, bv, cv):
        plan.run(da, bv, cv, stream=torch.cuda.current_stream().cuda_stream)
    got, pad, pad0 = strided_run(a, b, out_dtype, N + 64, N + 128, call)
    plan.close()
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(pad.view(np.uint8), pad0.view(np.uint8), err_msg="padding of C was written")


def test_sweep_graph_replays_match_eager(sweep):
    """The sweep kernel captured in a HIP graph: three replays with eager work
    in between, each equal to the eager result bit for bit."""
    import torch
    w = W.spmm_workload(4096, 4096, 1024, 32, 32, 0.05, seed=79)
    a = w["a"]
    plan = capi.SpmmPlan(bsr_of(a), 1024, "f32")
    assert plan.info()["persistent"] == 3
    da = torch.from_numpy(np.ascontiguousarray(a.data).view(np.int16)).cuda()
    db = torch.from_numpy(np.ascontiguousarray(w["b"]).view(np.int16)).cuda()
    eager = torch.empty((4096, 1024), dtype=torch.float32, device="cuda")
    plan.run(da, db, eager, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    out = torch.full((4096, 1024), float("nan"), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cap):
        plan.run(da, db, out, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref)
        plan.run(da, db, eager, stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    plan.close()
