"""ctypes binding of libbsparse (include/bsparse.h).

This is plumbing for Python callers (tests, bench.py): every compute call goes
to the HIP kernels in libbsparse.so.  There is no fallback: if the library is
missing, load() raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_int, c_int32, c_int64, c_void_p, c_char_p
from pathlib import Path
from typing import Optional

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libbsparse.so"
TIMELINE_PATH = PKG_DIR / "libbsparse_timeline.so"

ABI_VERSION = 6  # BSP_ABI_VERSION of include/bsparse.h
BSP_OK = 0
BSP_ERR_INVALID_ARGUMENT = 1
BSP_ERR_BAD_STRUCTURE = 2
BSP_ERR_UNSUPPORTED = 3
BSP_ERR_DEVICE = 4
BSP_ERR_OUT_OF_MEMORY = 5

DTYPE_F32 = 0
DTYPE_BF16 = 1
ROW_MAJOR = 0
COL_MAJOR = 1

# Every symbol include/bsparse.h declares, with (restype, argtypes).
_I32P = POINTER(c_int32)
_I64P = POINTER(c_int64)


class BsrDesc(ctypes.Structure):
    _fields_ = [
        ("H", c_int64),
        ("W", c_int64),
        ("R", c_int64),
        ("C", c_int64),
        ("nblocks", c_int64),
        ("indptr", _I32P),
        ("indices", _I32P),
    ]


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("kind", c_int32),
        ("tile_n", c_int32),
        ("n_tiles", c_int32),
        ("n_items", c_int32),
        ("n_entries", c_int32),
        ("n_split_rows", c_int32),
        ("n_slots", c_int32),
        ("grid", c_int32),
        ("max_item_entries", c_int32),
        ("stages", c_int32),
        ("group", c_int32),
        ("waves", c_int32),
        ("workspace_bytes", c_int64),
        ("persistent", c_int32),
        ("a_stages", c_int32),
        ("step_entries", c_int32),
        ("stripes_per_unit", c_int32),
        ("units_rotated", c_int32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_DESC_P = POINTER(BsrDesc)
_INFO_P = POINTER(PlanInfo)

SIGNATURES = {
    "bsp_abi_version": (c_int, []),
    "bsp_status_string": (c_char_p, [c_int]),
    "bsp_last_error": (c_char_p, []),
    "bsp_validate_bsr": (c_int, [_DESC_P]),
    "bsp_spmm_plan_create": (c_int, [POINTER(c_void_p), _DESC_P, c_int64, c_int, c_int, c_int]),
    "bsp_spmm": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "bsp_sddmm_plan_create": (c_int, [POINTER(c_void_p), _DESC_P, c_int64, c_int, c_int, c_int]),
    "bsp_sddmm": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "bsp_attention_plan_create": (c_int, [POINTER(c_void_p), _DESC_P, c_int64, c_int, c_int]),
    "bsp_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                              c_void_p, c_int64, c_void_p]),
    "bsp_plan_info_get": (c_int, [c_void_p, _INFO_P]),
    "bsp_plan_destroy": (c_int, [c_void_p]),
    "bsp_spmm_schedule": (c_int, [_DESC_P, c_int64, c_int, _INFO_P, _I32P, _I32P, _I64P, _I32P]),
    "bsp_sddmm_schedule": (c_int, [_DESC_P, c_int64, c_int, _INFO_P, _I32P, _I32P, _I64P, _I32P]),
    "bsp_spmm_sweep_schedule": (c_int, [_DESC_P, c_int64, c_int, c_int, _INFO_P, _I32P, _I32P, _I64P,
                                        POINTER(ctypes.c_uint32)]),
    "bsp_host_spmm": (c_int, [_DESC_P, c_void_p, c_void_p, c_int64, c_void_p, c_int, c_int]),
    "bsp_host_sddmm": (c_int, [_DESC_P, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int, c_int]),
    "bsp_spgemm_symbolic": (c_int, [_DESC_P, _DESC_P, _I64P, _I32P, _I32P]),
    "bsp_spgemm_plan_create": (c_int, [POINTER(c_void_p), _DESC_P, _DESC_P, c_int, c_int]),
    "bsp_spgemm_structure": (c_int, [c_void_p, _I64P, _I32P, _I32P]),
    "bsp_spgemm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "bsp_host_spgemm": (c_int, [_DESC_P, c_void_p, _DESC_P, c_void_p, _I32P, _I32P, c_void_p, c_int, c_int]),
    "bsp_spmm_noalloc": (c_int, [_DESC_P, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int, c_int,
                                 c_void_p]),
}
NOALLOC_SCRATCH_BYTES = 16 << 20  # BSP_NOALLOC_SCRATCH_BYTES of include/bsparse.h

_lib: Optional[ctypes.CDLL] = None


class BsparseError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"bsparse status {status}: {message}")
        self.status = status
        self.message = message


def load(path: Optional[Path] = None, force_reload: bool = False) -> ctypes.CDLL:
    """Loads libbsparse.so and declares every entry point; raises if absent."""
    global _lib
    if _lib is not None and path is None and not force_reload:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} not found: build it with __graft_entry__.build() "
            "(the HIP kernels are the only implementation)")
    # One HIP runtime per process: torch loads its own libamdhip64 (by the
    # name libamdhip64.so, through its RPATH), so if this library came first
    # with ROCm's libamdhip64.so.7, the process would hold two runtimes and
    # torch would find no GPU.  Loaded after torch, this library's
    # libamdhip64.so.7 resolves to torch's copy (same soname).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if a declared symbol is missing
        fn.restype = res
        fn.argtypes = args
    if lib.bsp_abi_version() != ABI_VERSION:
        raise ImportError(f"{p}: ABI version {lib.bsp_abi_version()}, this binding expects {ABI_VERSION}; "
                          "rebuild with __graft_entry__.build()")
    if path is None:
        _lib = lib
    return lib


def last_error(lib: Optional[ctypes.CDLL] = None) -> str:
    return (lib or load()).bsp_last_error().decode()


def check(status: int, lib: Optional[ctypes.CDLL] = None) -> None:
    if status != BSP_OK:
        raise BsparseError(status, last_error(lib))


TIMELINE_SLOTS = 64  # BSP_TIMELINE_SLOTS of include/bsparse_timeline.h
# Skip switches of the instrumented build (BSP_SKIP_* of include/bsparse_timeline.h).
SKIP_SPARSE_READ = 1   # A of SpMM, the mask values of SDDMM
SKIP_DENSE_READ = 2    # B of SpMM, X of SDDMM
SKIP_DENSE2_READ = 4   # Y of SDDMM
SKIP_COMPUTE = 8
SKIP_WRITE = 16
_timeline_lib: Optional[ctypes.CDLL] = None


def load_timeline() -> ctypes.CDLL:
    """libbsparse_timeline.so: every entry point of libbsparse.so (same
    results), plus per-workgroup time stamps and the skip switches
    (include/bsparse_timeline.h).  Pass it as `lib` to the plan classes to
    run a plan through it."""
    global _timeline_lib
    if _timeline_lib is None:
        lib = load(TIMELINE_PATH)
        lib.bsp_timeline_attach.restype = c_int
        lib.bsp_timeline_attach.argtypes = [c_void_p, c_int64, c_int]
        lib.bsp_timeline_clock_khz.restype = c_int
        lib.bsp_timeline_clock_khz.argtypes = [c_int, POINTER(c_int)]
        lib.bsp_timeline_skip.restype = c_int
        lib.bsp_timeline_skip.argtypes = [c_int]
        _timeline_lib = lib
    return _timeline_lib


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


class Bsr:
    """BSR structure (the index half of bsr_matrix<T>,
    sparse_common/bsr_matrix.hpp:205-213)."""

    def __init__(self, H: int, W: int, R: int, C: int, indptr, indices):
        self.H, self.W, self.R, self.C = int(H), int(W), int(R), int(C)
        self.indptr = _i32(indptr)
        self.indices = _i32(indices)

    @property
    def nblocks(self) -> int:
        return int(self.indices.size)

    @property
    def nbrows(self) -> int:
        return self.H // self.R

    def desc(self, nblocks: Optional[int] = None) -> BsrDesc:
        d = BsrDesc()
        d.H, d.W, d.R, d.C = self.H, self.W, self.R, self.C
        d.nblocks = self.nblocks if nblocks is None else nblocks
        d.indptr = self.indptr.ctypes.data_as(_I32P)
        d.indices = self.indices.ctypes.data_as(_I32P) if self.indices.size else ctypes.cast(None, _I32P)
        return d


def validate(bsr: Bsr) -> int:
    d = bsr.desc()
    return load().bsp_validate_bsr(ctypes.byref(d))


def _ptr(x) -> Optional[int]:
    """Address of a torch tensor (or a raw device address given as an int)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _operand(x, name: str, esize: int, rows: int, cols: int, ld: Optional[int], device: int):
    """Checks a device operand of `rows` x `cols` elements of `esize` bytes
    with row stride `ld` (elements) and returns (address, ld).

    A torch tensor must live on the plan's GPU, hold elements of `esize`
    bytes, have unit stride along its last dimension and cover
    (rows - 1) * ld + cols elements from its first one; a 2-D tensor's row
    stride is its stride(0) unless `ld` is given (they must then agree).  A
    raw int is taken as a device address as is (the caller vouches for it).
    Host arrays are refused: the kernels would read them as device addresses."""
    if x is None:
        raise ValueError(f"{name}: a device tensor is required")
    if isinstance(x, int):
        return x, (ld if ld is not None else cols)
    if isinstance(x, np.ndarray):
        raise TypeError(f"{name}: a numpy array is host memory; pass a torch tensor on the GPU")
    if not hasattr(x, "data_ptr") or not hasattr(x, "is_cuda"):
        raise TypeError(f"{name}: expected a torch tensor, got {type(x).__name__}")
    if not x.is_cuda:
        raise ValueError(f"{name}: tensor is on {x.device}, not on a GPU")
    if x.device.index is not None and x.device.index != device:
        raise ValueError(f"{name}: tensor is on cuda:{x.device.index}, the plan on device {device}")
    if x.element_size() != esize:
        raise ValueError(f"{name}: elements of {x.element_size()} bytes, expected {esize}")
    if x.dim() >= 1 and x.numel() > 0 and x.stride(-1) != 1:
        raise ValueError(f"{name}: the last dimension must be contiguous (stride 1), got stride {x.stride(-1)}")
    if x.dim() == 2:
        if x.shape[1] < cols and rows > 1:
            raise ValueError(f"{name}: {x.shape[1]} columns, need {cols}")
        st0 = x.stride(0)
        if ld is None:
            ld = st0 if x.shape[0] > 1 else cols
        elif x.shape[0] > 1 and ld != st0:
            raise ValueError(f"{name}: ld = {ld} but the tensor's row stride is {st0}")
    elif ld is None:
        ld = cols
    if x.dim() > 2:
        raise ValueError(f"{name}: expected a 1-D or 2-D tensor")
    need = (rows - 1) * ld + cols if rows > 0 and cols > 0 else 0
    avail = x.untyped_storage().nbytes() // esize - x.storage_offset()
    if need > avail:
        raise ValueError(f"{name}: covers {avail} elements from its start, the operand needs {need}")
    return x.data_ptr(), ld


def _dtype_code(out_dtype) -> int:
    if out_dtype in ("f32", "float32", DTYPE_F32):
        return DTYPE_F32
    if out_dtype in ("bf16", "bfloat16", DTYPE_BF16):
        return DTYPE_BF16
    raise ValueError(f"unsupported output dtype {out_dtype!r}")


class _Plan:
    def __init__(self, lib: Optional[ctypes.CDLL] = None):
        self._h = c_void_p()
        self._lib = lib or load()

    @property
    def handle(self) -> c_void_p:
        if not self._h:
            raise RuntimeError("plan is destroyed")
        return self._h

    def info(self) -> dict:
        inf = PlanInfo()
        check(self._lib.bsp_plan_info_get(self.handle, ctypes.byref(inf)), self._lib)
        return inf.as_dict()

    def close(self) -> None:
        if self._h:
            self._lib.bsp_plan_destroy(self._h)
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SpmmPlan(_Plan):
    """Plan for C[M x N] = A (BSR) * B[K x N] on one device."""

    def __init__(self, bsr: Bsr, N: int, out_dtype="f32", device: int = 0, lib: Optional[ctypes.CDLL] = None):
        super().__init__(lib)
        self.bsr, self.N, self.out_dtype, self.device = bsr, int(N), _dtype_code(out_dtype), device
        d = bsr.desc()
        check(self._lib.bsp_spmm_plan_create(ctypes.byref(self._h), ctypes.byref(d), self.N, ROW_MAJOR,
                                          self.out_dtype, device), self._lib)

    def run(self, a_vals, b, c, ldb: Optional[int] = None, ldc: Optional[int] = None,
            stream: Optional[int] = None) -> None:
        """a_vals: nblocks*R*C bf16; b: K x N bf16; c: M x N fp32 or bf16 (as
        planned); torch tensors on the plan's GPU (row strides from stride(0))."""
        bs = self.bsr
        nv = bs.nblocks * bs.R * bs.C
        pa = _operand(a_vals, "a_vals", 2, 1, nv, nv, self.device)[0] if nv else _ptr(a_vals)
        pb, ldb = _operand(b, "b", 2, bs.W, self.N, ldb, self.device)
        pc, ldc = _operand(c, "c", 4 if self.out_dtype == DTYPE_F32 else 2, bs.H, self.N, ldc, self.device)
        check(self._lib.bsp_spmm(self.handle, pa, pb, ldb, pc, ldc, stream), self._lib)


class SddmmPlan(_Plan):
    """Plan for out = mask (.) (X[M x K] * Y[K x N]) at the mask's blocks."""

    def __init__(self, mask: Bsr, K: int, y_layout: int = ROW_MAJOR, out_dtype="f32", device: int = 0, lib: Optional[ctypes.CDLL] = None):
        super().__init__(lib)
        self.mask, self.K, self.y_layout, self.device = mask, int(K), int(y_layout), device
        self.out_dtype = _dtype_code(out_dtype)
        d = mask.desc()
        check(self._lib.bsp_sddmm_plan_create(ctypes.byref(self._h), ctypes.byref(d), self.K, self.y_layout,
                                           self.out_dtype, device), self._lib)

    def run(self, mask_vals, x, y, out_vals, ldx: Optional[int] = None, ldy: Optional[int] = None,
            stream: Optional[int] = None) -> None:
        """mask_vals: nblocks*R*C bf16; x: M x K bf16; y: K x N (ROW_MAJOR) or
        N x K (COL_MAJOR) bf16; out_vals: nblocks*R*C fp32 or bf16; torch
        tensors on the plan's GPU."""
        m = self.mask
        nv = m.nblocks * m.R * m.C
        if nv == 0:
            check(self._lib.bsp_sddmm(self.handle, None, None, 0, None, 0, None, stream), self._lib)
            return
        pm = _operand(mask_vals, "mask_vals", 2, 1, nv, nv, self.device)[0]
        px, ldx = _operand(x, "x", 2, m.H, self.K, ldx, self.device)
        yr, yc = (self.K, m.W) if self.y_layout == ROW_MAJOR else (m.W, self.K)
        py, ldy = _operand(y, "y", 2, yr, yc, ldy, self.device)
        po = _operand(out_vals, "out_vals", 4 if self.out_dtype == DTYPE_F32 else 2, 1, nv, nv, self.device)[0]
        check(self._lib.bsp_sddmm(self.handle, pm, px, ldx, py, ldy, po, stream), self._lib)


class AttentionPlan(_Plan):
    """Plan for the fused pair O = bf16(mask (.) (Q * K^T)) * V on the mask's
    structure (queries x keys), head dimension 32, 64 or 128."""

    def __init__(self, mask: Bsr, head_dim: int, out_dtype="f32", device: int = 0, lib: Optional[ctypes.CDLL] = None):
        super().__init__(lib)
        self.mask, self.d, self.out_dtype, self.device = mask, int(head_dim), _dtype_code(out_dtype), device
        dsc = mask.desc()
        check(self._lib.bsp_attention_plan_create(ctypes.byref(self._h), ctypes.byref(dsc), self.d,
                                               self.out_dtype, device), self._lib)

    def run(self, mask_vals, q, k, v, out, ldq: Optional[int] = None, ldk: Optional[int] = None,
            ldv: Optional[int] = None, ldo: Optional[int] = None, stream: Optional[int] = None) -> None:
        """mask_vals: nblocks*R*C bf16; q: queries x d, k and v: keys x d bf16;
        out: queries x d fp32 or bf16; torch tensors on the plan's GPU."""
        m, d = self.mask, self.d
        nv = m.nblocks * m.R * m.C
        pm = _operand(mask_vals, "mask_vals", 2, 1, nv, nv, self.device)[0] if nv else _ptr(mask_vals)
        pq, ldq = _operand(q, "q", 2, m.H, d, ldq, self.device)
        pk, ldk = _operand(k, "k", 2, m.W, d, ldk, self.device)
        pv, ldv = _operand(v, "v", 2, m.W, d, ldv, self.device)
        po, ldo = _operand(out, "out", 4 if self.out_dtype == DTYPE_F32 else 2, m.H, d, ldo, self.device)
        check(self._lib.bsp_attention(self.handle, pm, pq, ldq, pk, ldk, pv, ldv, po, ldo, stream), self._lib)


def _structure(fn, nbrows: int, *args):
    """Runs a two-call structure query (NULL arrays for the size, then the
    arrays) and returns (indptr, indices)."""
    n = c_int64(0)
    null32 = ctypes.cast(None, _I32P)
    check(fn(*args, ctypes.byref(n), null32, null32))
    indptr = np.zeros(nbrows + 1, np.int32)
    indices = np.zeros(max(n.value, 1), np.int32)
    check(fn(*args, ctypes.byref(n), indptr.ctypes.data_as(_I32P), indices.ctypes.data_as(_I32P)))
    return indptr, indices[: n.value]


def spgemm_symbolic(a: Bsr, b: Bsr) -> Bsr:
    """Structure of A * B (host only): a Bsr of H x B.W in R x B.C blocks."""
    da, db = a.desc(), b.desc()
    indptr, indices = _structure(load().bsp_spgemm_symbolic, a.nbrows, ctypes.byref(da), ctypes.byref(db))
    return Bsr(a.H, b.W, a.R, b.C, indptr, indices)


class SpgemmPlan(_Plan):
    """Plan for C = A * B with A, B and C in BSR; `structure` is C's."""

    def __init__(self, a: Bsr, b: Bsr, out_dtype="f32", device: int = 0, lib: Optional[ctypes.CDLL] = None):
        super().__init__(lib)
        self.a, self.b, self.out_dtype, self.device = a, b, _dtype_code(out_dtype), device
        da, db = a.desc(), b.desc()
        check(self._lib.bsp_spgemm_plan_create(ctypes.byref(self._h), ctypes.byref(da), ctypes.byref(db),
                                            self.out_dtype, device), self._lib)
        indptr, indices = _structure(self._lib.bsp_spgemm_structure, a.nbrows, self.handle)
        self.structure = Bsr(a.H, b.W, a.R, b.C, indptr, indices)

    @property
    def out_values(self) -> int:
        return self.structure.nblocks * self.a.R * self.b.C

    def run(self, a_vals, b_vals, out_vals, stream: Optional[int] = None) -> None:
        """a_vals, b_vals: the operands' block values (bf16); out_vals:
        out_values fp32 or bf16; torch tensors on the plan's GPU."""
        na, nb, no = self.a.nblocks * self.a.R * self.a.C, self.b.nblocks * self.b.R * self.b.C, self.out_values
        pa = _operand(a_vals, "a_vals", 2, 1, na, na, self.device)[0] if na else _ptr(a_vals)
        pb = _operand(b_vals, "b_vals", 2, 1, nb, nb, self.device)[0] if nb else _ptr(b_vals)
        po = _operand(out_vals, "out_vals", 4 if self.out_dtype == DTYPE_F32 else 2, 1, no, no, self.device)[0] \
            if no else _ptr(out_vals)
        check(self._lib.bsp_spgemm(self.handle, pa, pb, po, stream), self._lib)


def _schedule(fn_name: str, bsr: Bsr, n: int, num_cus: int) -> dict:
    lib = load()
    fn = getattr(lib, fn_name)
    d = bsr.desc()
    inf = PlanInfo()
    null32, null64 = ctypes.cast(None, _I32P), ctypes.cast(None, _I64P)
    check(fn(ctypes.byref(d), n, num_cus, ctypes.byref(inf), null32, null32, null64, null32))
    items = np.zeros((max(inf.n_items, 1), 6), np.int32)
    ent_row = np.zeros(max(inf.n_entries, 1), np.int32)
    ent_off = np.zeros(max(inf.n_entries, 1), np.int64)
    wgmap = np.zeros(max(inf.grid, 1), np.int32)
    check(fn(ctypes.byref(d), n, num_cus, ctypes.byref(inf), items.ctypes.data_as(_I32P),
             ent_row.ctypes.data_as(_I32P), ent_off.ctypes.data_as(_I64P), wgmap.ctypes.data_as(_I32P)))
    return {
        "info": inf.as_dict(),
        "items": items[: inf.n_items],
        "ent_row": ent_row[: inf.n_entries],
        "ent_off": ent_off[: inf.n_entries],
        "wgmap": wgmap[: inf.grid],
    }


def spmm_schedule(bsr: Bsr, N: int, num_cus: int = 256) -> dict:
    return _schedule("bsp_spmm_schedule", bsr, N, num_cus)


def spmm_sweep_schedule(bsr: Bsr, N: int, num_cus: int = 256, col_groups: int = 0) -> dict:
    """The sweep kernel's schedule (host only): per-workgroup records
    {first entry, entries, first sweep, sweeps}, sweep records {entries,
    stripe of slots 0-15, first column of slots 0-15}, and the entry words."""
    lib = load()
    d = bsr.desc()
    inf = PlanInfo()
    null32, null64 = ctypes.cast(None, _I32P), ctypes.cast(None, _I64P)
    nullu = ctypes.cast(None, POINTER(ctypes.c_uint32))
    check(lib.bsp_spmm_sweep_schedule(ctypes.byref(d), N, num_cus, col_groups, ctypes.byref(inf), null32, null32,
                                      null64, nullu))
    wgs = np.zeros((max(inf.grid, 1), 4), np.int32)
    sweeps = np.zeros((max(inf.n_slots, 1), 33), np.int32)
    bw = np.zeros(max(inf.n_entries, 1), np.int64)
    aw = np.zeros(max(inf.n_entries, 1), np.uint32)
    check(lib.bsp_spmm_sweep_schedule(ctypes.byref(d), N, num_cus, col_groups, ctypes.byref(inf),
                                      wgs.ctypes.data_as(_I32P), sweeps.ctypes.data_as(_I32P),
                                      bw.ctypes.data_as(_I64P), aw.ctypes.data_as(POINTER(ctypes.c_uint32))))
    return {"info": inf.as_dict(), "wgs": wgs[: inf.grid], "sweeps": sweeps[: inf.n_slots],
            "bw": bw[: inf.n_entries], "aw": aw[: inf.n_entries]}


def sddmm_schedule(mask: Bsr, K: int, num_cus: int = 256) -> dict:
    return _schedule("bsp_sddmm_schedule", mask, K, num_cus)


def host_spmm(bsr: Bsr, a_vals: np.ndarray, b: np.ndarray, out_dtype="f32", device: int = 0) -> np.ndarray:
    """Blocking host-buffer SpMM (the HostCodeFunctionPtr shape)."""
    code = _dtype_code(out_dtype)
    a_vals = np.ascontiguousarray(a_vals, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    N = b.shape[1]
    out = np.empty((bsr.H, N), np.float32 if code == DTYPE_F32 else np.uint16)
    d = bsr.desc()
    check(load().bsp_host_spmm(ctypes.byref(d), a_vals.ctypes.data, b.ctypes.data, N, out.ctypes.data,
                               code, device))
    return out


def host_sddmm(mask: Bsr, mask_vals: np.ndarray, x: np.ndarray, y: np.ndarray, out_dtype="f32",
               device: int = 0) -> np.ndarray:
    """Blocking host-buffer SDDMM (the SDDMMHostCodeFunctionPtr shape); returns block values."""
    code = _dtype_code(out_dtype)
    mask_vals = np.ascontiguousarray(mask_vals, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.uint16)
    y = np.ascontiguousarray(y, dtype=np.uint16)
    K = x.shape[1]
    out = np.empty(mask.nblocks * mask.R * mask.C, np.float32 if code == DTYPE_F32 else np.uint16)
    d = mask.desc()
    check(load().bsp_host_sddmm(ctypes.byref(d), mask_vals.ctypes.data, x.ctypes.data, y.ctypes.data, K,
                                out.ctypes.data, code, device))
    return out


def host_spgemm(a: Bsr, a_vals: np.ndarray, b: Bsr, b_vals: np.ndarray, out_dtype="f32", device: int = 0):
    """Blocking host-buffer SpGEMM (bsr_matrix<T>::spgemm's shape): returns
    (structure Bsr, block values)."""
    code = _dtype_code(out_dtype)
    st = spgemm_symbolic(a, b)
    a_vals = np.ascontiguousarray(a_vals, dtype=np.uint16)
    b_vals = np.ascontiguousarray(b_vals, dtype=np.uint16)
    indptr = np.zeros(a.nbrows + 1, np.int32)
    indices = np.zeros(max(st.nblocks, 1), np.int32)
    out = np.empty(max(st.nblocks * a.R * b.C, 1), np.float32 if code == DTYPE_F32 else np.uint16)
    da, db = a.desc(), b.desc()
    check(load().bsp_host_spgemm(ctypes.byref(da), a_vals.ctypes.data, ctypes.byref(db), b_vals.ctypes.data,
                                 indptr.ctypes.data_as(_I32P), indices.ctypes.data_as(_I32P), out.ctypes.data,
                                 code, device))
    return Bsr(a.H, b.W, a.R, b.C, indptr, indices[: st.nblocks]), out[: st.nblocks * a.R * b.C]

