"""The C++ host mirror (bsr_matrix / dense_matrix / HostCodeFunctionPtr-shaped
entry points) through the reference-shaped test drivers in tests/cpp."""
import subprocess

import pytest

from helpers import REPO

BUILD = REPO / "tests" / "cpp" / "_build"


def _tool(name):
    exe = BUILD / name
    if not exe.exists():  # built by __graft_entry__.build(); build here only if missing
        subprocess.run(["make", "-s", "-C", str(REPO / "tests" / "cpp")], check=True, capture_output=True)
    return str(exe)


def _run(args, timeout):
    p = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    print(p.stdout[-4000:])
    return p


@pytest.mark.parametrize("rotate", ["1", "0"])
def test_scheduler_work_lists(rotate):
    """tests/cpp/test_schedule: the host scheduler's SpMM, SDDMM and SpGEMM
    work lists and workgroup maps (built from the scheduler's source with g++;
    make rebuilds it when the source changed), with the persistent units
    rotated by column group (the default) and in CSR order (BSP_SPMM_ROTATE=0)."""
    import os
    subprocess.run(["make", "-s", "-C", str(REPO / "tests" / "cpp"), "_build/test_schedule"], check=True,
                   capture_output=True)
    env = dict(os.environ, BSP_SPMM_ROTATE=rotate)
    p = subprocess.run([str(BUILD / "test_schedule")], capture_output=True, text=True, timeout=120, env=env)
    print(p.stdout[-4000:])
    assert p.returncode == 0, p.stdout + p.stderr
    assert "PASS (0 failed checks)" in p.stdout


def test_sddmm_cpu_only_structure_mode():
    """test_sddmm <all> -1: the reference's device-free mode (structure only)."""
    p = _run([_tool("test_sddmm"), "-1", "-1"], 120)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "Passed: 17 / 17" in p.stdout


def test_block_spmm_lists_registry():
    p = _run([_tool("test_block_spmm"), "list"], 120)
    assert p.returncode == 0 and "test_1_block_id" in p.stdout


@pytest.mark.gpu
def test_block_spmm_registry_on_gpu():
    p = _run([_tool("test_block_spmm"), "all", "0"], 600)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert "FAIL" not in p.stdout


@pytest.mark.gpu
def test_sddmm_registry_on_gpu():
    p = _run([_tool("test_sddmm"), "-1", "0"], 300)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert "Passed: 17 / 17" in p.stdout


def test_spgemm_cpu_only_structure_mode():
    """test_spgemm <all> -1: the symbolic phase against the oracle's structure."""
    p = _run([_tool("test_spgemm"), "-1", "-1"], 120)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "Passed: 10 / 10" in p.stdout


@pytest.mark.gpu
def test_spgemm_host_mirror_on_gpu():
    p = _run([_tool("test_spgemm"), "-1", "0"], 300)
    assert p.returncode == 0, p.stdout[-3000:] + p.stderr[-2000:]
    assert "Passed: 10 / 10" in p.stdout


def test_build_fails_on_kernels_that_spill():
    """The build reads the compiler's kernel-resource-usage remarks and stops
    at any kernel with a nonzero ScratchSize (a kernel that spills runs far
    below its roofline without any other sign)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bsp_build", REPO / "tenstorrent-wh-blockspmm_amd" / "build.py")
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)
    clean = ("remark: k.hip:1:0: Function Name: _Z1av [-Rpass-analysis=kernel-resource-usage]\n"
             "remark: k.hip:1:0:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n")
    build.check_no_scratch(clean, "k.hip")
    spill = clean + ("remark: k.hip:9:0: Function Name: _Z1bv [-Rpass-analysis=kernel-resource-usage]\n"
                     "remark: k.hip:9:0:     ScratchSize [bytes/lane]: 132 [-Rpass-analysis=kernel-resource-usage]\n")
    with pytest.raises(RuntimeError, match=r"_Z1bv: 132 bytes/lane"):
        build.check_no_scratch(spill, "k.hip")
