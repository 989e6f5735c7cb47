"""SpMM and SDDMM launches captured in a HIP graph (as bench.py times them):
every replay, with eager work in between, equals the eager result bit for bit.
The skewed case captures both the SpMM kernel and the split-row reduction."""
import numpy as np
import pytest

from helpers import W, bsr_of, capi

pytestmark = pytest.mark.gpu


def _dev(torch, arr):
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).to("cuda")


@pytest.mark.parametrize("kernel,split", [("persistent", None), ("items", None), ("items", 5)])
def test_spmm_graph_replays_match_eager(monkeypatch, kernel, split):
    import torch
    if kernel == "items":
        monkeypatch.setenv("BSP_SPMM_STREAM", "0")
    if split:
        monkeypatch.setenv("BSP_SPMM_SPLIT", str(split))
    w = W.spmm_workload(2048, 2048, 512, 32, 32, 0.1, seed=31)
    a = w["a"]
    plan = capi.SpmmPlan(bsr_of(a), 512, "f32")
    assert plan.info()["persistent"] == (kernel == "persistent")
    if split:
        assert plan.info()["n_split_rows"] > 0
    da, db = _dev(torch, a.data), _dev(torch, w["b"])
    eager = torch.empty((2048, 512), dtype=torch.float32, device="cuda")
    plan.run(da, db, eager, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    out = torch.full((2048, 512), float("nan"), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cap):
        plan.run(da, db, out, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))          # eager work between replays
        _ = (db.float() * 2).sum().item()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"replay {rep}")
    plan.close()


def test_sddmm_graph_replays_match_eager():
    import torch
    s = W.workload_sddmm(M=1024, N=1024, K=128, density=0.2, seed=32)
    m = s["mask"]
    plan = capi.SddmmPlan(bsr_of(m), 128, capi.ROW_MAJOR, "f32")
    dm, dx, dy = _dev(torch, m.data), _dev(torch, s["x"]), _dev(torch, s["y"])
    n = m.nblocks * 1024
    eager = torch.empty(n, dtype=torch.float32, device="cuda")
    plan.run(dm, dx, dy, eager, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    out = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cap):
        plan.run(dm, dx, dy, out, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"replay {rep}")
    plan.close()


@pytest.mark.parametrize("waves", [4, 8])
def test_graph_keeps_the_plans_kernel_after_an_environment_change(monkeypatch, waves):
    """The wave count of the 256-column row-group kernel is fixed when the plan
    is created: a graph captured from that plan, replayed after the
    environment asks for the other count, still runs the plan's kernel and
    gives the eager result bit for bit."""
    import torch
    monkeypatch.setenv("BSP_SPMM_WIDE_WAVES", str(waves))
    monkeypatch.setenv("BSP_SPMM_GROUP", "4")
    monkeypatch.setenv("BSP_SPMM_WIDE_GROUP", "2")
    w = W.spmm_workload(2048, 2048, 512, 128, 128, 0.25, seed=33)
    a = w["a"]
    plan = capi.SpmmPlan(bsr_of(a), 512, "f32")
    assert plan.info()["waves"] == waves and plan.info()["group"] == 4
    da, db = _dev(torch, a.data), _dev(torch, w["b"])
    eager = torch.empty((2048, 512), dtype=torch.float32, device="cuda")
    plan.run(da, db, eager, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    out = torch.full((2048, 512), float("nan"), dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=cap):
        plan.run(da, db, out, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    monkeypatch.setenv("BSP_SPMM_WIDE_WAVES", str(12 - waves))
    assert plan.info()["waves"] == waves
    for rep in range(2):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"replay {rep}")
    # an eager launch after the change also keeps the plan's kernel
    plan.run(da, db, out, stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    plan.close()
