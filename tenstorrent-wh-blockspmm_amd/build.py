"""Builds libbsparse.so (HIP kernels for gfx950 + C ABI) in place, and beside
it libbsparse_timeline.so (the same sources with BSP_TIMELINE: every entry
point of libbsparse.so, plus per-workgroup time stamps, include/
bsparse_timeline.h) and libbsp_probe.so (memory-system probes for bench.py).

Run as a script or through build_library().  The libraries are written next to
this file; tests, bench.py and the C++ host tools load them from there.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO / "include"
LIB_PATH = PKG_DIR / "libbsparse.so"
TIMELINE_PATH = PKG_DIR / "libbsparse_timeline.so"
PROBE_PATH = PKG_DIR / "libbsp_probe.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in device code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

SOURCES = ["bsp_kernels.hip", "bsp_capi.cpp", "bsp_schedule.cpp", "bsp_noalloc.hip"]


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, cwd=str(PKG_DIR), capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")
    return proc.stderr


def check_no_scratch(remarks: str, src: str) -> None:
    """Fails the build when a kernel of `src` spills to scratch memory (the
    compiler's kernel-resource-usage remarks report ScratchSize per kernel)."""
    spills, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            spills.append(f"{name}: {m.group(1)} bytes/lane")
    if spills:
        raise RuntimeError(f"{src}: kernels spill to scratch:\n  " + "\n  ".join(spills))


def _compile(src: str, obj: Path, defines: list[str], verbose: bool) -> str:
    lang = ["-x", "hip", "-Rpass-analysis=kernel-resource-usage"] if src.endswith(".hip") else []
    cmd = [HIPCC, *HIP_FLAGS, *defines, f"-I{INCLUDE}", f"-I{CSRC}", *lang, "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd))
    remarks = _run(cmd)
    if src.endswith(".hip"):
        check_no_scratch(remarks, src + (" (" + " ".join(defines) + ")" if defines else ""))
    return str(obj)


def _link(objs: list[str], out: Path, verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, out)


def build_library(verbose: bool = False) -> Path:
    """Compiles every source (in parallel) and links libbsparse.so,
    libbsparse_timeline.so and libbsp_probe.so; always rebuilds."""
    from concurrent.futures import ThreadPoolExecutor
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; libbsparse.so needs ROCm's hipcc for gfx950")
    build_dir = PKG_DIR / "_build"
    (build_dir / "timeline").mkdir(parents=True, exist_ok=True)
    plain = [(src, build_dir / (src + ".o"), []) for src in SOURCES]
    timed = [(src, build_dir / "timeline" / (src + ".o"), ["-DBSP_TIMELINE"]) for src in SOURCES]
    probe = [("bsp_probe.hip", build_dir / "bsp_probe.hip.o", [])]
    # the kernel files first: they take the longest
    jobs = sorted(plain + timed + probe, key=lambda j: not j[0].startswith("bsp_kernels"))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(lambda j: _compile(j[0], j[1], j[2], verbose), jobs))
    _link([str(j[1]) for j in plain], LIB_PATH, verbose)
    _link([str(j[1]) for j in timed], TIMELINE_PATH, verbose)
    # The memory-system probe bench.py uses for the on-chip roof (a library of
    # its own: it is not part of the boundary).
    _link([str(j[1]) for j in probe], PROBE_PATH, verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
