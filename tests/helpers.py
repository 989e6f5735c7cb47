"""Shared test helpers: package/oracle loading, device runners through the C
ABI, and the parity criterion."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO))
import __graft_entry__ as entry  # noqa: E402

pkg = entry.load_package()
capi = pkg.capi
W = pkg.workloads
orc = entry._load_oracle()

# Host threads for the oracle: the GPU box gives one GPU's share (16 cores).
ORACLE_THREADS = min(16, os.cpu_count() or 1)


def bsr_of(a) -> "capi.Bsr":
    return capi.Bsr(a.H, a.W, a.R, a.C, a.indptr, a.indices)


# ---------------------------------------------------------------------------
# Parity criterion.
def tolerance(golden: np.ndarray, k_eff) -> np.ndarray:
    """Elementwise bound |y - g| <= 1e-2 * sqrt(K_e / 32) * max(1, |g|), with
    K_e the reduction length of the element (SpMM: stored blocks in the row
    times C; SDDMM: K)."""
    k = np.maximum(np.asarray(k_eff, dtype=np.float64), 32.0)
    return 1e-2 * np.sqrt(k / 32.0) * np.maximum(1.0, np.abs(golden.astype(np.float64)))


def spmm_k_eff(a) -> np.ndarray:
    """Reduction length per output row: C times the blocks stored in its block row."""
    return np.repeat(np.diff(a.indptr).astype(np.int64) * a.C, a.R)[:, None]


def compare(got: np.ndarray, golden: np.ndarray, k_eff) -> dict:
    got = np.asarray(got, dtype=np.float64)
    g = np.asarray(golden, dtype=np.float64)
    err = np.abs(got - g)
    bound = tolerance(g, k_eff)
    finite = np.isfinite(got).all()
    rel = err / np.maximum(np.abs(g), 1e-30)
    res = {
        "ok": bool(finite and np.all(err <= bound)),
        "max_abs": float(err.max()) if err.size else 0.0,
        "max_rel_over_1": float((err / np.maximum(1.0, np.abs(g))).max()) if err.size else 0.0,
        "max_rel": float(rel[np.abs(g) > 1e-3].max()) if (np.abs(g) > 1e-3).any() else 0.0,
        "worst_ratio": float((err / bound).max()) if err.size else 0.0,
        "finite": bool(finite),
    }
    if g.size > 1 and np.std(g) > 0:
        res["pcc"] = orc.pcc(got.astype(np.float32), g.astype(np.float32))
    return res


def assert_parity(got, golden, k_eff, what=""):
    res = compare(got, golden, k_eff)
    assert res["ok"], f"{what}: parity failed {res}"
    return res


# ---------------------------------------------------------------------------
# Device runners (C ABI, device pointers on torch's current stream).
def _dev_u16(arr: np.ndarray):
    import torch
    arr = np.ascontiguousarray(arr, dtype=np.uint16)
    if arr.size == 0:
        return torch.zeros(8, dtype=torch.int16, device="cuda")
    return torch.from_numpy(arr.view(np.int16)).to("cuda")


def run_spmm(a, b: np.ndarray, out_dtype="f32", plan=None, poison=True) -> np.ndarray:
    """C = A*B on the GPU; returns fp32 (bf16 outputs widened exactly)."""
    import torch
    M, N = a.H, b.shape[1]
    own = plan is None
    if own:
        plan = capi.SpmmPlan(bsr_of(a), N, out_dtype)
    da = _dev_u16(a.data if a.data is not None else np.zeros(0, np.uint16))
    db = _dev_u16(b)
    if out_dtype == "f32":
        dc = torch.full((M, N), float("nan") if poison else 0.0, dtype=torch.float32, device="cuda")
    else:
        dc = torch.full((M, N), 0x7FC0 if poison else 0, dtype=torch.int16, device="cuda")
    plan.run(da, db, dc, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = dc.cpu().numpy()
    if own:
        plan.close()
    if out_dtype == "f32":
        return out
    return W.bf16_to_f32(out.view(np.uint16))


def strided_run(a, b, out_dtype, ldb, ldc, call):
    """Runs `call(da, b_view, c_view)` with B and C as the first N columns of
    wider tensors (row strides ldb and ldc), their padding poisoned with NaN.
    Returns (C as fp32, C's padding as raw bits, the padding's poison bits)."""
    import torch
    K, N, M = a.W, b.shape[1], a.H
    da = torch.from_numpy(np.ascontiguousarray(a.data).view(np.int16)).cuda()
    bw = torch.full((K, ldb), 0x7FC0, dtype=torch.int16, device="cuda")
    bw[:, :N] = torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).cuda()
    if out_dtype == "f32":
        cw = torch.full((M, ldc), float("nan"), dtype=torch.float32, device="cuda")
    else:
        cw = torch.full((M, ldc), 0x7FC0, dtype=torch.int16, device="cuda")
    pad0 = cw[:, N:].cpu().numpy().copy()
    call(da, bw[:, :N], cw[:, :N])
    torch.cuda.synchronize()
    out = cw.cpu().numpy()
    got = out[:, :N] if out_dtype == "f32" else W.bf16_to_f32(out[:, :N].view(np.uint16))
    return np.ascontiguousarray(got), out[:, N:], pad0


def run_sddmm(mask, x: np.ndarray, y: np.ndarray, out_dtype="f32", y_layout=None, plan=None,
              poison=True) -> np.ndarray:
    """mask (.) (X*Y) block values on the GPU; y is passed as given (K x N for
    ROW_MAJOR, N x K for COL_MAJOR)."""
    import torch
    if y_layout is None:
        y_layout = capi.ROW_MAJOR
    K = x.shape[1]
    own = plan is None
    if own:
        plan = capi.SddmmPlan(bsr_of(mask), K, y_layout, out_dtype)
    nv = mask.nblocks * mask.R * mask.C
    dm = _dev_u16(mask.data)
    dx = _dev_u16(x)
    dy = _dev_u16(y)
    if out_dtype == "f32":
        do = torch.full((max(nv, 1),), float("nan") if poison else 0.0, dtype=torch.float32, device="cuda")
    else:
        do = torch.full((max(nv, 1),), 0x7FC0 if poison else 0, dtype=torch.int16, device="cuda")
    ldy = mask.W if y_layout == capi.ROW_MAJOR else K
    plan.run(dm, dx, dy, do, ldy=ldy, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = do.cpu().numpy()[:nv]
    if own:
        plan.close()
    if out_dtype == "f32":
        return out
    return W.bf16_to_f32(out.view(np.uint16))


def golden_spmm(a, b, threads=ORACLE_THREADS) -> np.ndarray:
    return orc.spmm(a.indptr, a.indices, a.data, a.H, a.W, a.R, a.C, b, threads=threads)


def golden_sddmm(mask, x, y, y_colmajor=False, threads=ORACLE_THREADS) -> np.ndarray:
    return orc.sddmm(mask.indptr, mask.indices, mask.data, mask.H, mask.W, mask.R, mask.C, x, y,
                     y_colmajor=y_colmajor, threads=threads)


def with_values(s, content="RAND", seed=0):
    """Attaches block values of a content type to a structure."""
    rng = np.random.default_rng(seed)
    s.data = W.block_content(s.nblocks, s.R, s.C, content, rng)
    return s


def run_attention(mask, q: np.ndarray, k: np.ndarray, v: np.ndarray, out_dtype="f32", plan=None,
                  poison=True) -> np.ndarray:
    """Fused O = bf16(mask (.) Q K^T) V on the GPU; returns fp32."""
    import torch
    d = q.shape[1]
    own = plan is None
    if own:
        plan = capi.AttentionPlan(bsr_of(mask), d, out_dtype)
    dm, dq, dk, dv = _dev_u16(mask.data), _dev_u16(q), _dev_u16(k), _dev_u16(v)
    M = mask.H
    if out_dtype == "f32":
        do = torch.full((M, d), float("nan") if poison else 0.0, dtype=torch.float32, device="cuda")
    else:
        do = torch.full((M, d), 0x7FC0 if poison else 0, dtype=torch.int16, device="cuda")
    plan.run(dm, dq, dk, dv, do, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = do.cpu().numpy()
    if own:
        plan.close()
    if out_dtype == "f32":
        return out
    return W.bf16_to_f32(out.view(np.uint16))


def golden_attention(mask, q, k, v):
    """The oracle chain: S = mask (.) Q K^T (SDDMM with K as column-major Y),
    rounded to bf16, then O = S V (SpMM on the mask's structure).  Returns
    (O, S as BSR arrays)."""
    s = golden_sddmm(mask, q, k, y_colmajor=True)
    a = W.BsrArrays(mask.H, mask.W, mask.R, mask.C, mask.indptr, mask.indices, W.bf16_from_f32(s))
    return golden_spmm(a, v), a


def block_pattern(s) -> np.ndarray:
    """Stored-block counts per (block row, block column) (duplicates counted)."""
    p = np.zeros((s.H // s.R, s.W // s.C), np.int64)
    rows = np.repeat(np.arange(s.H // s.R), np.diff(s.indptr))
    np.add.at(p, (rows, s.indices), 1)
    return p


def spgemm_k_eff(a, b, structure) -> np.ndarray:
    """Reduction length per output value of A*B: the (A, B) block pairs that
    meet at the output block times the shared block width C."""
    pairs = block_pattern(a) @ block_pattern(b)
    rows = np.repeat(np.arange(structure.H // structure.R), np.diff(structure.indptr))
    per_block = pairs[rows, structure.indices] * a.C
    return np.repeat(per_block, a.R * b.C)


def golden_spgemm(a, b):
    """(indptr, indices, fp32 values) of the oracle's BSR x BSR product."""
    return orc.spgemm(a.indptr, a.indices, a.data, a.H, a.R, a.C, b.indptr, b.indices, b.data, b.W, b.C)


def run_spgemm(a, b, out_dtype="f32", plan=None, poison=True):
    """A*B on the GPU: (structure as capi.Bsr, values widened to fp32)."""
    import torch
    own = plan is None
    if own:
        plan = capi.SpgemmPlan(bsr_of(a), bsr_of(b), out_dtype)
    da, db = _dev_u16(a.data), _dev_u16(b.data)
    nv = plan.out_values
    if out_dtype == "f32":
        do = torch.full((max(nv, 1),), float("nan") if poison else 0.0, dtype=torch.float32, device="cuda")
    else:
        do = torch.full((max(nv, 1),), 0x7FC0 if poison else 0, dtype=torch.int16, device="cuda")
    plan.run(da, db, do, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = do.cpu().numpy()[:nv]
    st = plan.structure
    if own:
        plan.close()
    if out_dtype == "f32":
        return st, out
    return st, W.bf16_to_f32(out.view(np.uint16))
