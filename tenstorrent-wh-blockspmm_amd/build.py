"""Builds libbsparse.so (HIP kernels for gfx950 + C ABI) in place.

Run as a script or through build_library().  The library is written next to
this file; tests, bench.py and the C++ host tools load it from there.
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


def build_library(verbose: bool = False) -> Path:
    """Compiles every source and links libbsparse.so; always rebuilds."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; libbsparse.so needs ROCm's hipcc for gfx950")
    build_dir = PKG_DIR / "_build"
    build_dir.mkdir(exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = build_dir / (src + ".o")
        lang = ["-x", "hip", "-Rpass-analysis=kernel-resource-usage"] if src.endswith(".hip") else []
        cmd = [HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *lang, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        remarks = _run(cmd)
        if src.endswith(".hip"):
            check_no_scratch(remarks, src)
        objs.append(str(obj))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, LIB_PATH)
    # The memory-system probe bench.py uses for the on-chip roof (a library of
    # its own: it is not part of the boundary).
    obj = build_dir / "bsp_probe.hip.o"
    _run([HIPCC, *HIP_FLAGS, "-x", "hip", "-c", str(CSRC / "bsp_probe.hip"), "-o", str(obj)])
    tmp = PROBE_PATH.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", str(obj), "-o", str(tmp)])
    os.replace(tmp, PROBE_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
