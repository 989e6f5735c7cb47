"""bench.py's result line, built from stub timings on the CPU: one compact
JSON object (well under what the round's driver records) carrying the
headline keys, the HBM roofline and the CPU baseline of the skewed 16384^2
workload, and one summary row per configuration."""
import importlib.util
import json

import pytest

from helpers import REPO

spec = importlib.util.spec_from_file_location("bench_mod", REPO / "bench.py")
bench = importlib.util.module_from_spec(spec)
spec.loader.exec_module(bench)

REQUIRED = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def _rec(us, flops, nbytes, kernel_us=None, traffic=None, cpu=True, **extra):
    t = {"launch_ms": us * 1e-3, "kernel_us": kernel_us,
         "kernels": {"void bsp::spmm_stream_kernel<1, 14, 16, 4, 1, false, 2, 1>(bsp::SpmmStreamArgs)":
                     {"median_us": kernel_us, "mean_us": kernel_us, "launches": 20}} if kernel_us else {}}
    r = bench.summarize(t, flops, nbytes)
    if traffic:
        r["traffic"] = {"bytes_per_launch": traffic, "ratio_to_algorithmic": round(traffic / nbytes, 3),
                        "source": "profiles/x.md", "kernel": "k"}
    if cpu:
        r["cpu"] = {"single": {"tflops": 0.0012, "cores": 1, "seconds": 0.4, "sample": "block rows 0..9 (80 blocks)",
                               "gpu_speedup": 1e5},
                    "all": {"tflops": 0.012, "cores": 16, "seconds": 0.9, "sample": "whole workload",
                            "gpu_speedup": 1e4},
                    "kind": "port"}
    r.update(extra)
    return r


def _stub_sections():
    out = {"c1": _rec(3.5, 5.35e7, 1.76e6, 3.0, 3.27e6)}
    sweep = []
    for d, nnzb in ((0.01, 164), (0.05, 819), (0.25, 4096), (0.5, 8192)):
        for od in ("f32", "bf16"):
            r = _rec(13.2, 2.0 * nnzb * 1024 * 512, 21e6, 12.0, 43e6,
                     plan={"tile_n": 128, "n_entries": nnzb * 4, "grid": 512})
            r.update({"density": d, "out": od})
            sweep.append(r)
        sweep.append({"density": d, "out": "f32", "warm_cache": True, **bench.summarize({"launch_ms": 0.01}, 1e9, 1e7)})
    out["sweep"] = sweep
    out["sddmm"] = _rec(7.2, 8.6e8, 14.3e6, 7.1, 22.9e6)
    out["skewed"] = _rec(39.8, 1.0995e10, 111.4e6, 38.9, 255.9e6, nnzb=5243, max_row_blocks=107,
                         input_sha256="0" * 64)
    out["attention"] = {"sddmm": _rec(8.0, 7e8, 15e6, cpu=False), "spmm": _rec(6.0, 7e8, 12e6, cpu=False),
                        "fused": _rec(10.0, 1.4e9, 25e6, cpu=False), "cpu": out["c1"]["cpu"]}
    out["spgemm"] = {"runs": [dict(_rec(80.0, 2.7e9, 7.7e7, cpu=False), out=o) for o in ("f32", "bf16")]}
    out["large_blocks"] = {"runs": [dict(_rec(800.0, 2.7e11, 2.7e8, cpu=False), out=o) for o in ("bf16", "f32")]}
    out["block_sizes"] = {"runs": [dict(_rec(900.0, 2.7e11, 2.7e8, cpu=False), R=R) for R in (128, 64)]}
    pats = []
    for p, d in [(p, d) for d in (0.05, 0.5) for p in bench.PATTERNS] + [("tril", 0.5156), ("triu", 0.5156)]:
        pats.append(dict(_rec(500.0, 5.5e11, 3.3e8, cpu=False), pattern=p, density=d,
                         reference_dda_tflops_n150=48.0))
    out["patterns"] = {"runs": pats}
    out["host_entry"] = {"ms_per_call": 12.3}
    return out


ROOFS = {"l2_stream_tbs": 33.0, "hbm_stream_tbs": 5.6, "empty_launch_us": 1.77}


def test_headline_line_is_compact_and_complete():
    out = _stub_sections()
    big = {"tflops": 1300.0}
    line = bench.build_headline(out, ROOFS, big, 20, 5, "gpurun_out/bench_sections.json")
    text = json.dumps(line, separators=(",", ":"))
    assert len(text) < bench.HEADLINE_MAX_BYTES, len(text)
    back = json.loads(text)
    for k in REQUIRED:
        assert k in back, k
    assert back["n_gpus"] == 1 and back["steps"] == 20 and back["warmup"] == 5
    assert back["value"] == pytest.approx(1.0995e10 / 39.8e-6 / 1e12, rel=1e-3)
    assert back["ms_per_step"] == pytest.approx(0.0398)
    assert "16384x16384" in back["config"]["workload"]
    rl = back["roofline"]
    assert rl["bound"] == "hbm" and rl["unit"] == "GB/s" and rl["peak"] == bench.PEAK_HBM_GBS
    assert rl["achieved"] == pytest.approx(111.4e6 / 39.8e-6 / 1e9, rel=1e-3)
    assert rl["frac"] == pytest.approx(rl["achieved"] / rl["peak"], abs=1e-4)
    assert rl["traffic"] == 255.9e6
    assert rl["floor_us"] == pytest.approx(1.77 + 111.4e6 / 5.6e12 * 1e6, abs=1e-3)
    cpu = back["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["cores"] == 16 and cpu["unit"] == "TFLOP/s" and cpu["value"] > 0
    rows = back["summary"]
    for key in ("c1", "c2_1_f32", "c2_1_bf16", "c2_5_f32", "c2_25_f32", "c2_25_bf16", "c2_50_f32", "c2_50_bf16",
                "c3", "c4", "c5_sddmm", "c5_spmm", "c5_fused", "spgemm_f32", "8192c_256_bf16", "8192c_64_f32",
                "pat_row_5", "pat_tril", "host_ms"):
        assert key in rows, key
    for key in ("c1", "c2_1_f32", "c2_5_f32", "c3", "c4"):
        assert {"floor_us", "frac_of_floor", "us", "kernel_us", "traffic_x"} <= set(rows[key]), key
    assert "on_chip_frac" in rows["c2_25_f32"]
    assert rows["c4"]["cpu_x"] == [1e5, 1e4]


def test_headline_floor_takes_the_longer_roof():
    # bytes-bound and FLOP-bound launches
    assert bench.floor_us(1e9, 80e6, ROOFS) == pytest.approx(1.77 + 80e6 / 5.6e12 * 1e6, abs=1e-3)
    assert bench.floor_us(2.5e12, 1e6, ROOFS) == pytest.approx(1.77 + 1000.0, rel=1e-6)
