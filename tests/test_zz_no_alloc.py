"""bsp_spmm_noalloc (the SpMM entry point that allocates no device memory,
staging its schedule in the library's static device array) against bsp_spmm
with a plan, through the C ABI: two calls in a row, the second on a smaller
problem (the array keeps the first call's contents), each bit-identical to
the plan's result, which the oracle (block_spmm/inc/bsr_matrix.hpp:954-1000)
also checks."""
import ctypes

import numpy as np
import pytest

from helpers import W, assert_parity, bsr_of, capi, golden_spmm, run_spmm, spmm_k_eff

pytestmark = pytest.mark.gpu


def _noalloc(a, b, out_dtype):
    import torch
    M, N = a.H, b.shape[1]
    da = torch.from_numpy(np.ascontiguousarray(a.data).view(np.int16)).cuda()
    db = torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).cuda()
    if out_dtype == "f32":
        dc = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    else:
        dc = torch.full((M, N), 0x7FC0, dtype=torch.int16, device="cuda")
    bsr = bsr_of(a)
    d = bsr.desc()
    code = capi.DTYPE_F32 if out_dtype == "f32" else capi.DTYPE_BF16
    st = capi.load().bsp_spmm_noalloc(ctypes.byref(d), da.data_ptr(), db.data_ptr(), N, N, dc.data_ptr(), N, code, 0,
                                      torch.cuda.current_stream().cuda_stream)
    capi.check(st)
    torch.cuda.synchronize()
    out = dc.cpu().numpy()
    return out if out_dtype == "f32" else W.bf16_to_f32(out.view(np.uint16))


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_noalloc_matches_the_plan_on_two_calls_the_second_smaller(out_dtype):
    big = W.workload_spmm_sweep(0.25)          # 4096 x 4096, 4096 blocks, N = 512
    small = W.spmm_workload(1024, 2048, 256, 32, 32, 0.1, seed=97)   # 2048 x 256 x 1024
    for w in (big, small):
        got = _noalloc(w["a"], w["b"], out_dtype)
        ref = run_spmm(w["a"], w["b"], out_dtype)
        np.testing.assert_array_equal(got, ref)
        assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]), f"noalloc {out_dtype}")


def test_noalloc_skewed_and_empty_rows():
    """The skewed workload (rows of 1 .. 107 blocks, empty stripes among them),
    then an empty matrix: zeros everywhere, no stale tiles from the call before."""
    w = W.workload_spmm_skewed()
    np.testing.assert_array_equal(_noalloc(w["a"], w["b"], "f32"), run_spmm(w["a"], w["b"], "f32"))
    a = W.BsrArrays(1024, 1024, 32, 32, np.zeros(33, np.int32), np.zeros(0, np.int32))
    a.data = np.zeros(16, np.uint16)
    b = W.dense_content(1024, 128, "RAND", np.random.default_rng(3))
    assert np.all(_noalloc(a, b, "f32") == 0.0)
