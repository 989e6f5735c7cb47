"""bsparse for MI355X: block-sparse SpMM and SDDMM (bf16, fp32 accumulate) as
hand-written HIP kernels for gfx950 behind a C ABI (include/bsparse.h).

The directory name is not a Python identifier; import it through
load_package() in __graft_entry__.py (registered as ``bsparse_amd``).
"""
from . import capi, workloads  # noqa: F401

__all__ = ["capi", "workloads"]
