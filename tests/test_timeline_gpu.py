"""The profiling build (libbsparse_timeline.so: the same sources with
per-workgroup time stamps, include/bsparse_timeline.h) on the GPU: it gives
the same bits as libbsparse.so (it skips no work), on the persistent SpMM of
the 4096^2 25% workload, the skewed 16384^2 workload (persistent and sweep
kernels) and the one-shot SDDMM, and its stamps are ordered: start <= first
landing <= end, per workgroup.  The reference's counterpart is its profiling
registry (block_spmm/inc/host_code.hpp:195-222)."""
import numpy as np
import pytest

from helpers import W, bsr_of, capi, run_sddmm, run_spmm

pytestmark = pytest.mark.gpu


def _stamps_ok(stamps):
    s = stamps.astype(np.int64)
    live = s[:, 0] > 0
    assert live.sum() > 0
    s = s[live]
    assert np.all(s[:, 63] >= s[:, 0])
    landed = s[:, 1] > 0
    assert np.all(s[landed, 1] >= s[landed, 0]) and np.all(s[landed, 63] >= s[landed, 1])
    # every workgroup's stamps within a second of each other (100 MHz clock)
    assert (s[:, 63].max() - s[:, 0].min()) < 100_000_000


def _spmm_through(lib, a, b, out_dtype, monkeypatch, env):
    import torch
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    plan = capi.SpmmPlan(bsr_of(a), b.shape[1], out_dtype, lib=lib)
    info = plan.info()
    stamps = None
    if lib is not capi.load():
        stamps = torch.zeros((info["grid"], capi.TIMELINE_SLOTS), dtype=torch.int64, device="cuda")
        capi.check(lib.bsp_timeline_attach(stamps.data_ptr(), info["grid"], 0), lib)
    try:
        out = run_spmm(a, b, out_dtype, plan=plan)
    finally:
        if stamps is not None:
            lib.bsp_timeline_attach(None, 0, 0)
    plan.close()
    for k in env:
        monkeypatch.delenv(k)
    return out, (stamps.cpu().numpy() if stamps is not None else None), info


@pytest.mark.parametrize("case,env", [("c2_25", {}), ("c4", {}), ("c4", {"BSP_SPMM_SWEEP": "2"}),
                                      ("c4", {"BSP_SPMM_BALANCE": "0"})])
def test_timeline_build_gives_the_same_bits(monkeypatch, case, env):
    w = W.workload_spmm_sweep(0.25) if case == "c2_25" else W.workload_spmm_skewed()
    tl = capi.load_timeline()
    ref, _, info0 = _spmm_through(capi.load(), w["a"], w["b"], "f32", monkeypatch, env)
    got, stamps, info1 = _spmm_through(tl, w["a"], w["b"], "f32", monkeypatch, env)
    assert info0 == info1
    np.testing.assert_array_equal(got, ref)
    _stamps_ok(stamps)
    if info1["persistent"] in (1, 2) and case == "c4":
        # one stamp per unit with entries (slots 2 ..), in stream order
        units = stamps[:, 2:63]
        assert (units > 0).sum() > 0
        for row in units:
            v = row[row > 0]
            assert np.all(np.diff(v.astype(np.int64)) >= 0)


def test_timeline_build_sddmm_same_bits():
    import torch
    s = W.workload_sddmm()
    m = s["mask"]
    ref = run_sddmm(m, s["x"], s["y"], "f32")
    tl = capi.load_timeline()
    plan = capi.SddmmPlan(bsr_of(m), s["K"], capi.ROW_MAJOR, "f32", lib=tl)
    grid = plan.info()["grid"]
    stamps = torch.zeros((grid, capi.TIMELINE_SLOTS), dtype=torch.int64, device="cuda")
    capi.check(tl.bsp_timeline_attach(stamps.data_ptr(), grid, 0), tl)
    try:
        got = run_sddmm(m, s["x"], s["y"], "f32", plan=plan)
    finally:
        tl.bsp_timeline_attach(None, 0, 0)
    plan.close()
    np.testing.assert_array_equal(got, ref)
    st = stamps.cpu().numpy()
    _stamps_ok(st)
    live = st[:, 0] > 0
    assert np.all(st[live, 2] >= st[live, 1])  # products after the operands landed


# ---- skip switches (bsp_timeline_skip) -------------------------------------
# The reference's profiling variants leave a part of the work out
# (block_spmm/inc/host_code.hpp:86-153: _no_a_read, _no_b_read, _no_compute,
# _no_write; block_sddmm/inc/host_code.hpp:71-101).  Here each switch is run
# on every kernel that has it: the launch completes, a skipped write leaves
# the NaN-poisoned output untouched, skipped products store zeros, and with
# the switches cleared the same plan gives the plain library's bits again.
SPMM_SWITCH_CASES = [
    ("persistent 4096^2 25%", lambda: W.workload_spmm_sweep(0.25), {}),
    ("sweep 4096^2 25%", lambda: W.workload_spmm_sweep(0.25), {"BSP_SPMM_SWEEP": "2"}),
    ("row groups 4096^2 256x256 25% N=2048", lambda: W.spmm_workload(4096, 4096, 2048, 256, 256, 0.25, 7), {}),
]


@pytest.fixture
def switches():
    tl = capi.load_timeline()
    yield tl
    capi.check(tl.bsp_timeline_skip(0), tl)


@pytest.mark.parametrize("label,make,env", SPMM_SWITCH_CASES, ids=[c[0] for c in SPMM_SWITCH_CASES])
def test_spmm_skip_switches(monkeypatch, switches, label, make, env):
    tl = switches
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    w = make()
    a, b = w["a"], w["b"]
    ref = run_spmm(a, b, "f32")
    plan = capi.SpmmPlan(bsr_of(a), b.shape[1], "f32", lib=tl)
    info = plan.info()
    if "sweep" in label:
        assert info["persistent"] == 3
    elif "row groups" in label:
        assert info["persistent"] == 0 and info["group"] > 1 and info["tile_n"] == 256
    else:
        assert info["persistent"] in (1, 2)
    try:
        for flags in (capi.SKIP_SPARSE_READ, capi.SKIP_DENSE_READ, capi.SKIP_COMPUTE, capi.SKIP_WRITE,
                      capi.SKIP_SPARSE_READ | capi.SKIP_DENSE_READ | capi.SKIP_COMPUTE | capi.SKIP_WRITE):
            capi.check(tl.bsp_timeline_skip(flags), tl)
            out = run_spmm(a, b, "f32", plan=plan)
            if flags & capi.SKIP_WRITE:
                assert np.isnan(out).all(), flags
            elif flags == capi.SKIP_COMPUTE:
                assert (out == 0).all()
        capi.check(tl.bsp_timeline_skip(0), tl)
        np.testing.assert_array_equal(run_spmm(a, b, "f32", plan=plan), ref)
    finally:
        plan.close()


def test_sddmm_skip_switches(switches):
    tl = switches
    s = W.workload_sddmm()
    m = s["mask"]
    ref = run_sddmm(m, s["x"], s["y"], "f32")
    plan = capi.SddmmPlan(bsr_of(m), s["K"], capi.ROW_MAJOR, "f32", lib=tl)
    try:
        for flags in (capi.SKIP_SPARSE_READ, capi.SKIP_DENSE_READ, capi.SKIP_DENSE2_READ, capi.SKIP_COMPUTE,
                      capi.SKIP_WRITE, 31):
            capi.check(tl.bsp_timeline_skip(flags), tl)
            out = run_sddmm(m, s["x"], s["y"], "f32", plan=plan)
            if flags & capi.SKIP_WRITE:
                assert np.isnan(out).all(), flags
            elif flags == capi.SKIP_COMPUTE:
                assert (out == 0).all()
            elif flags == capi.SKIP_SPARSE_READ:
                assert (out == 0).all()  # the mask values read as zero
        capi.check(tl.bsp_timeline_skip(0), tl)
        np.testing.assert_array_equal(run_sddmm(m, s["x"], s["y"], "f32", plan=plan), ref)
    finally:
        plan.close()


def test_skip_switches_refused_by_kernels_without_them(switches):
    """A per-item 32x32 SpMM plan (BSP_SPMM_STREAM=0) has no switches: with
    flags set its launch is refused, not run whole."""
    import os
    tl = switches
    w = W.workload_spmm_sweep(0.05)
    os.environ["BSP_SPMM_STREAM"] = "0"
    try:
        plan = capi.SpmmPlan(bsr_of(w["a"]), w["b"].shape[1], "f32", lib=tl)
    finally:
        del os.environ["BSP_SPMM_STREAM"]
    try:
        assert plan.info()["persistent"] == 0 and plan.info()["group"] == 1
        capi.check(tl.bsp_timeline_skip(capi.SKIP_WRITE), tl)
        with pytest.raises(capi.BsparseError) as ei:
            run_spmm(w["a"], w["b"], "f32", plan=plan)
        assert ei.value.status == capi.BSP_ERR_UNSUPPORTED
    finally:
        plan.close()
