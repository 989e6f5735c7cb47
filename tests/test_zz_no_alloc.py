"""bsp_spmm_noalloc (the SpMM entry point that allocates no device memory,
staging its schedule in the library's static device array) against bsp_spmm
with a plan, through the C ABI: two calls in a row, the second on a smaller
problem (the array keeps the first call's contents), each bit-identical to
the plan's result, which the oracle (block_spmm/inc/bsr_matrix.hpp:954-1000)
also checks."""
import ctypes

import numpy as np
import pytest

from helpers import W, assert_parity, bsr_of, capi, golden_spmm, run_spmm, spmm_k_eff, strided_run

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


def _noalloc_call(a, N, out_dtype):
    import torch
    code = capi.DTYPE_F32 if out_dtype == "f32" else capi.DTYPE_BF16
    bsr = bsr_of(a)
    d = bsr.desc()

    def call(da, bv, cv):
        st = capi.load().bsp_spmm_noalloc(ctypes.byref(d), da.data_ptr(), bv.data_ptr(), N, bv.stride(0),
                                          cv.data_ptr(), cv.stride(0), code, 0, torch.cuda.current_stream().cuda_stream)
        capi.check(st)
    return call, bsr


@pytest.mark.parametrize("out_dtype", ["f32", "bf16"])
def test_noalloc_strided_b_and_c(out_dtype):
    """B and C as column slices of wider tensors (ldb = N + 64, ldc = N + 128,
    padding poisoned with NaN): equal to the contiguous no-allocation call bit
    for bit, held to the oracle, padding untouched."""
    w = W.spmm_workload(2048, 2048, 512, 32, 32, 0.1, seed=92)
    a, b = w["a"], w["b"]
    N = b.shape[1]
    call, keep = _noalloc_call(a, N, out_dtype)
    got, pad, pad0 = strided_run(a, b, out_dtype, N + 64, N + 128, call)
    np.testing.assert_array_equal(got, _noalloc(a, b, out_dtype))
    np.testing.assert_array_equal(pad.view(np.uint8), pad0.view(np.uint8), err_msg="padding of C was written")
    assert_parity(got, golden_spmm(a, b), spmm_k_eff(a), f"noalloc strided {out_dtype}")
    del keep


@pytest.mark.parametrize("R", [64, 128])
def test_noalloc_large_blocks_held_to_the_oracle(R):
    """Blocks of R = C = 64 and 128 (a plan may take a row-group kernel for
    them, summing in another order): the no-allocation call runs the 32-row
    persistent kernel and is held to the oracle, not to the plan's bits."""
    w = W.spmm_workload(1024, 2048, 512, R, R, 0.2, seed=93 + R)
    for od in ("f32", "bf16"):
        got = _noalloc(w["a"], w["b"], od)
        assert_parity(got, golden_spmm(w["a"], w["b"]), spmm_k_eff(w["a"]), f"noalloc R={R} {od}")
