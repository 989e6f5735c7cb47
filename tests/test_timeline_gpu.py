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
