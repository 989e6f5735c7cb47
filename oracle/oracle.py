"""ORACLE binding — test infrastructure, not product code.

numpy wrappers over liboracle.so (bsp_oracle.c, the C restatement of the
reference's CPU golden).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, and only as the checker (bench.py also
times it as the CPU baseline).
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_uint16
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_lib = None


def build() -> Path:
    """Compiles liboracle.so with the committed Makefile (gcc, -O3, OpenMP)."""
    subprocess.run(["make", "-s", "-B", "-C", str(ORACLE_DIR), "liboracle.so"], check=True,
                   capture_output=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    p32, pu16, pf = POINTER(c_int32), POINTER(c_uint16), POINTER(c_float)
    lib.orc_spmm_bf16.argtypes = [p32, p32, pu16, c_int64, c_int64, c_int64, pu16, c_int64, c_int64,
                                  pf, c_int, c_int]
    lib.orc_spmm_bf16.restype = c_int
    lib.orc_sddmm.argtypes = [p32, p32, pu16, c_int64, c_int64, c_int64, pu16, c_int64, pu16, c_int64,
                              c_int, pf, c_int, c_int]
    lib.orc_sddmm.restype = c_int
    lib.orc_spgemm.argtypes = [p32, p32, pu16, c_int64, c_int64, c_int64, p32, p32, pu16, c_int64,
                               c_int64, p32, p32, pf, POINTER(c_int64), c_int]
    lib.orc_spgemm.restype = c_int
    lib.orc_bsr_to_dense.argtypes = [p32, p32, pu16, c_int64, c_int64, c_int64, c_int64, pu16]
    lib.orc_bsr_to_dense.restype = c_int
    lib.orc_gemm_bf16.argtypes = [pu16, pu16, c_int64, c_int64, c_int64, pf]
    lib.orc_gemm_bf16.restype = c_int
    lib.orc_pcc.argtypes = [pf, pf, c_int64]
    lib.orc_pcc.restype = c_float
    lib.orc_bf16_from_f32_array.argtypes = [pf, pu16, c_int64]
    lib.orc_bf16_to_f32_array.argtypes = [pu16, pf, c_int64]
    lib.orc_have_openmp.restype = c_int
    _lib = lib
    return lib


def _p(a, t):
    return a.ctypes.data_as(POINTER(t))


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def spmm(indptr, indices, a_vals, H, W, R, C, b, threads: int = 1, mutation: int = 0) -> np.ndarray:
    """fp32 golden of C = A*B (block_spmm/inc/bsr_matrix.hpp:954-1000)."""
    indptr, indices, a_vals, b = _i32(indptr), _i32(indices), _u16(a_vals), _u16(b)
    K, N = b.shape
    assert K == W
    out = np.empty((H, N), np.float32)
    idx = indices if indices.size else np.zeros(1, np.int32)
    av = a_vals if a_vals.size else np.zeros(1, np.uint16)
    rc = load().orc_spmm_bf16(_p(indptr, c_int32), _p(idx, c_int32), _p(av, c_uint16), H // R, R, C,
                              _p(b, c_uint16), K, N, _p(out, c_float), threads, mutation)
    assert rc == 0
    return out


def sddmm(indptr, indices, mask_vals, H, W, R, C, x, y, y_colmajor: bool = False, threads: int = 1,
          mutation: int = 0) -> np.ndarray:
    """fp32 golden of mask (.) (X*Y) block values (sparse_common/bsr_matrix.hpp:816-857)."""
    indptr, indices, mask_vals, x, y = _i32(indptr), _i32(indices), _u16(mask_vals), _u16(x), _u16(y)
    K = x.shape[1]
    nblocks = int(indptr[-1])
    out = np.empty(max(nblocks * R * C, 1), np.float32)
    idx = indices if indices.size else np.zeros(1, np.int32)
    mv = mask_vals if mask_vals.size else np.zeros(1, np.uint16)
    rc = load().orc_sddmm(_p(indptr, c_int32), _p(idx, c_int32), _p(mv, c_uint16), H // R, R, C,
                          _p(x, c_uint16), K, _p(y, c_uint16), W, int(y_colmajor), _p(out, c_float),
                          threads, mutation)
    assert rc == 0
    return out[: nblocks * R * C]


def spgemm(a_indptr, a_indices, a_vals, H, R, C, b_indptr, b_indices, b_vals, BW, BC,
           mutation: int = 0):
    """fp32 golden of BSR x BSR -> BSR (sparse_common/bsr_matrix.hpp:741-810):
    returns (indptr, indices, values[nblocks*R*BC])."""
    a_indptr, a_indices, a_vals = _i32(a_indptr), _i32(a_indices), _u16(a_vals)
    b_indptr, b_indices, b_vals = _i32(b_indptr), _i32(b_indices), _u16(b_vals)
    nbr, nbc = H // R, BW // BC
    lib = load()
    ai = a_indices if a_indices.size else np.zeros(1, np.int32)
    av = a_vals if a_vals.size else np.zeros(1, np.uint16)
    bi = b_indices if b_indices.size else np.zeros(1, np.int32)
    bv = b_vals if b_vals.size else np.zeros(1, np.uint16)
    indptr = np.zeros(nbr + 1, np.int32)
    n = c_int64(0)
    args = [_p(a_indptr, c_int32), _p(ai, c_int32), _p(av, c_uint16), nbr, R, C, _p(b_indptr, c_int32),
            _p(bi, c_int32), _p(bv, c_uint16), BC, nbc, _p(indptr, c_int32)]
    assert lib.orc_spgemm(*args, None, None, ctypes.byref(n), mutation) == 0
    indices = np.zeros(max(n.value, 1), np.int32)
    vals = np.zeros(max(n.value * R * BC, 1), np.float32)
    assert lib.orc_spgemm(*args, _p(indices, c_int32), _p(vals, c_float), ctypes.byref(n), mutation) == 0
    return indptr, indices[: n.value], vals[: n.value * R * BC]


def to_dense(indptr, indices, vals, H, W, R, C) -> np.ndarray:
    """bf16 dense expansion (sparse_common/bsr_matrix.hpp:1056-1070)."""
    indptr, indices, vals = _i32(indptr), _i32(indices), _u16(vals)
    out = np.empty((H, W), np.uint16)
    idx = indices if indices.size else np.zeros(1, np.int32)
    v = vals if vals.size else np.zeros(1, np.uint16)
    assert load().orc_bsr_to_dense(_p(indptr, c_int32), _p(idx, c_int32), _p(v, c_uint16), H // R, R, C,
                                   W, _p(out, c_uint16)) == 0
    return out


def gemm(a, b) -> np.ndarray:
    """fp32-accumulated dense GEMM of bf16 inputs (sparse_common/bsr_matrix.hpp:158-171)."""
    a, b = _u16(a), _u16(b)
    H, K = a.shape
    W = b.shape[1]
    out = np.empty((H, W), np.float32)
    assert load().orc_gemm_bf16(_p(a, c_uint16), _p(b, c_uint16), H, K, W, _p(out, c_float)) == 0
    return out


def pcc(x, y) -> float:
    """Pearson r as check_bfloat16_vector_pcc computes it (sparse_common/bmm_op.hpp:79-113)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.ascontiguousarray(y, dtype=np.float32).ravel()
    return float(load().orc_pcc(_p(x, c_float), _p(y, c_float), x.size))


def bf16_from_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    load().orc_bf16_from_f32_array(_p(x, c_float), _p(out, c_uint16), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    load().orc_bf16_to_f32_array(_p(h, c_uint16), _p(out, c_float), h.size)
    return out


def have_openmp() -> bool:
    return bool(load().orc_have_openmp())
