"""The sweep kernel's host schedule (bsp_spmm_sweep_schedule), on the CPU:
every 32x32 sub-block product of every (stripe, 128-column tile) unit appears
exactly once, each unit sits in exactly one slot of one sweep of one
workgroup, sweeps hold at most 16 units and an even number of entries (a
skip entry pads an odd one), entries of a sweep ascend in block column,
the entry words agree with the slot records, and each unit's last entry in
stream order (only it) carries the last bit.  The reference's host analysis
this replaces for such shapes: block_spmm/inc/host_code/
bsr_spmm_multicore_load_balanced_new_DM.cpp:339-393."""
import numpy as np
import pytest

from helpers import W, bsr_of, capi

SKIP = 1 << 60
LAST = 1 << 61


def _expected(a, N):
    """{(stripe, n0, block, k-sub)} of every sub-block product."""
    RS, CS = a.R // 32, a.C // 32
    out = set()
    rows = np.repeat(np.arange(a.nbrows), np.diff(a.indptr))
    for blk in range(a.nblocks):
        i = int(rows[blk])
        for sub in range(RS):
            for t in range(CS):
                for n0 in range(0, N, 128):
                    out.add((i * RS + sub, n0, blk, t))
    return out


def _check(a, N, num_cus=256, col_groups=0):
    s = capi.spmm_sweep_schedule(bsr_of(a), N, num_cus, col_groups)
    info, wgs, sweeps, bw, aw = s["info"], s["wgs"], s["sweeps"], s["bw"], s["aw"]
    RS, CS = a.R // 32, a.C // 32
    rows = np.repeat(np.arange(a.nbrows), np.diff(a.indptr))
    assert info["persistent"] == 3 and info["grid"] == len(wgs) == (num_cus // 8) * 8
    seen, units = [], []
    for g, (w0, n, s0, ns) in enumerate(wgs):
        assert n % 2 == 0
        e = w0
        for r in range(s0, s0 + ns):
            rec = sweeps[r]
            cnt, srows, sn0 = int(rec[0]), rec[1:17], rec[17:33]
            assert cnt % 2 == 0
            live = srows >= 0
            assert 1 <= live.sum() <= 16
            units += [(int(srows[j]), int(sn0[j])) for j in range(16) if live[j]]
            words = bw[e:e + cnt]
            brow = words & 0xFFFFFFFF
            assert np.all(np.diff(brow[(words & SKIP) == 0]) >= 0), "a sweep's entries ascend in block column"
            # the last bit marks exactly each unit's final entry in stream order, never a skip entry
            live_words = [int(wd) for wd in words if not wd & SKIP]
            assert not any(int(wd) & LAST for wd in words if wd & SKIP)
            final = {}
            for i, wd in enumerate(live_words):
                final[(wd >> 56) & 15] = i
            assert {i for i, wd in enumerate(live_words) if wd & LAST} == set(final.values())
            for wd, av in zip(words, aw[e:e + cnt]):
                if wd & SKIP:
                    continue
                slot = (int(wd) >> 56) & 15
                n0 = (int(wd) >> 32) & 0xFFFFFF
                stripe = int(srows[slot])
                assert stripe >= 0 and n0 == int(sn0[slot])
                off = int(av) * 32
                blk, rem = divmod(off, a.R * a.C)
                sub, t = rem // (32 * a.C), (rem % a.C) // 32
                assert stripe == int(rows[blk]) * RS + sub
                assert int(wd & 0xFFFFFFFF) == int(a.indices[blk]) * a.C + 32 * t
                seen.append((stripe, n0, blk, t))
            e += cnt
        assert e == w0 + n
    assert len(seen) == len(set(seen)), "a product appears twice"
    assert set(seen) == _expected(a, N)
    all_units = {(sr, n0) for sr in range(a.H // 32) for n0 in range(0, N, 128)}
    assert len(units) == len(set(units)) and set(units) == all_units
    return s


def test_sweep_schedule_skewed_workload():
    """The skewed 16384^2 x 1024 workload: 4096 units over 256 workgroups,
    one sweep each, the column-group count of least estimated reads."""
    w = W.workload_spmm_skewed()
    s = _check(w["a"], 1024)
    assert s["info"]["n_items"] == 4096
    assert (s["wgs"][:, 3] == 1).all()


@pytest.mark.parametrize("cg", [1, 2, 4, 8])
def test_sweep_schedule_column_groups(cg):
    a = W.spmm_workload(4096, 4096, 1024, 32, 32, 0.05, seed=61)["a"]
    s = _check(a, 1024, col_groups=cg)
    assert s["info"]["group"] == cg


def test_sweep_schedule_several_sweeps_and_empty_rows():
    """More units than 16 per workgroup (several sweeps), a third of the
    block rows empty (sweeps of zero tiles among them), on 64 compute units."""
    rng = np.random.default_rng(62)
    a = W.random_positions(4096, 4096, 32, 32, 2000, W.Rng(63))
    keep = rng.random(a.nbrows) > 0.33
    ptr, idx = [0], []
    for i in range(a.nbrows):
        if keep[i]:
            idx += list(a.indices[a.indptr[i]:a.indptr[i + 1]])
        ptr.append(len(idx))
    b = W.BsrArrays(4096, 4096, 32, 32, np.array(ptr, np.int32), np.array(idx, np.int32))
    s = _check(b, 1024, num_cus=64)
    assert s["info"]["n_slots"] > len(s["wgs"])


@pytest.mark.parametrize("R,C", [(64, 64), (32, 128), (128, 32)])
def test_sweep_schedule_larger_blocks(R, C):
    a = W.random_positions(2048, 2048, R, C, 300, W.Rng(64 + R + C))
    _check(a, 512)


def test_sweep_schedule_unsorted_and_duplicate_columns():
    """Rows with shuffled and repeated block columns (the reference's FILL_COL
    yields such rows): every copy is its own product."""
    rng = np.random.default_rng(65)
    ptr, idx = [0], []
    for i in range(128):
        cols = list(rng.choice(128, size=int(rng.integers(0, 12)), replace=False))
        cols += [c for c in cols if rng.random() < 0.3]
        rng.shuffle(cols)
        idx += cols
        ptr.append(len(idx))
    a = W.BsrArrays(4096, 4096, 32, 32, np.array(ptr, np.int32), np.array(idx, np.int32))
    _check(a, 256)


def test_sweep_schedule_rejects_unsupported_shapes():
    a = W.random_positions(1024, 1024, 32, 32, 100, W.Rng(66))
    with pytest.raises(capi.BsparseError):
        capi.spmm_sweep_schedule(bsr_of(a), 96)
    b = W.BsrArrays(1024, 1024, 16, 16, np.zeros(65, np.int32), np.zeros(0, np.int32))
    with pytest.raises(capi.BsparseError):
        capi.spmm_sweep_schedule(bsr_of(b), 128)


def test_sweep_schedule_without_load_balancing(monkeypatch):
    """BSP_SPMM_BALANCE=0: stripes onto row groups and units onto workgroups
    in contiguous ranges; still every product once."""
    monkeypatch.setenv("BSP_SPMM_BALANCE", "0")
    w = W.workload_spmm_skewed()
    s = _check(w["a"], 1024)
    n = s["wgs"][:, 1]
    assert n.max() > 2 * n.mean()  # the skew shows without balancing
