"""C ABI on the CPU: the library loads and exports every declared entry point,
malformed input is rejected with the documented status before any device
work, and the host-side schedule covers every sub-block product exactly once
with balanced pieces.  No compute call needs a GPU here."""
import ctypes
import re
import subprocess

import numpy as np
import pytest

from helpers import REPO, W, bsr_of, capi

HEADER = REPO / "include" / "bsparse.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bsp_[a-z_0-9]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = _declared_functions()
    assert len(names) >= 14
    lib = capi.load()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(capi.SIGNATURES), "binding and header disagree"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(capi.LIB_PATH)], capture_output=True, text=True)
    exported = set(re.findall(r"\bT (bsp_\w+)", nm.stdout))
    assert set(names) <= exported


def test_timeline_library_exports_the_same_entry_points_and_its_own():
    """libbsparse_timeline.so (the profiling build) exports every function of
    bsparse.h and the three of bsparse_timeline.h; the skip switches take
    only the BSP_SKIP_* bits (set and cleared here without a device)."""
    lib = capi.load_timeline()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    text = re.sub(r"/\*.*?\*/", "", (REPO / "include" / "bsparse_timeline.h").read_text(), flags=re.S)
    own = sorted(set(re.findall(r"\b(bsp_[a-z_0-9]+)\s*\(", text)))
    assert own == ["bsp_timeline_attach", "bsp_timeline_clock_khz", "bsp_timeline_skip"]
    for name in own:
        assert hasattr(lib, name)
    assert lib.bsp_timeline_attach(None, 5, 0) == capi.BSP_ERR_INVALID_ARGUMENT
    flags = dict(re.findall(r"#define (BSP_SKIP_\w+) (\d+)", text))
    assert {k: int(v) for k, v in flags.items()} == {
        "BSP_SKIP_SPARSE_READ": capi.SKIP_SPARSE_READ, "BSP_SKIP_DENSE_READ": capi.SKIP_DENSE_READ,
        "BSP_SKIP_DENSE2_READ": capi.SKIP_DENSE2_READ, "BSP_SKIP_COMPUTE": capi.SKIP_COMPUTE,
        "BSP_SKIP_WRITE": capi.SKIP_WRITE}
    assert lib.bsp_timeline_skip(32) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_timeline_skip(-1) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_timeline_skip(31) == capi.BSP_OK
    assert lib.bsp_timeline_skip(0) == capi.BSP_OK
    assert not hasattr(capi.load(), "bsp_timeline_skip")  # the plain library has no switches


def test_library_links_hip_and_has_gfx950_code():
    out = subprocess.run(["ldd", str(capi.LIB_PATH)], capture_output=True, text=True).stdout
    assert "libamdhip64" in out
    blob = capi.LIB_PATH.read_bytes()
    assert b"gfx950" in blob
    assert b"oracle" not in blob.lower().replace(b"_oracle", b"")  # never linked against the oracle


def test_abi_version_and_status_strings():
    lib = capi.load()
    assert lib.bsp_abi_version() == capi.ABI_VERSION == 6
    for code, text in [(0, b"ok"), (2, b"malformed BSR structure"), (3, b"unsupported")]:
        assert lib.bsp_status_string(code) == text


def _bsr(indptr, indices, H=128, Wd=128, R=32, C=32):
    return capi.Bsr(H, Wd, R, C, np.array(indptr, np.int32), np.array(indices, np.int32))


GOOD = dict(indptr=[0, 1, 1, 3, 3], indices=[2, 0, 3])

BAD = [
    ("indptr0", dict(indptr=[1, 1, 1, 3, 3], indices=[2, 0, 3]), capi.BSP_ERR_BAD_STRUCTURE, "indptr[0]"),
    ("decreasing", dict(indptr=[0, 2, 1, 3, 3], indices=[2, 0, 3]), capi.BSP_ERR_BAD_STRUCTURE, "non-decreasing"),
    ("last", dict(indptr=[0, 1, 1, 2, 2], indices=[2, 0, 3]), capi.BSP_ERR_BAD_STRUCTURE, "nblocks"),
    ("col_range", dict(indptr=[0, 1, 1, 3, 3], indices=[2, 0, 4]), capi.BSP_ERR_BAD_STRUCTURE, "outside"),
    ("col_negative", dict(indptr=[0, 1, 1, 3, 3], indices=[2, -1, 3]), capi.BSP_ERR_BAD_STRUCTURE, "outside"),
]


def test_validate_accepts_good_and_duplicate_columns():
    assert capi.validate(_bsr(**GOOD)) == capi.BSP_OK
    dup = W.fill_col_as_reference(64, 64, 32, 32, 4)
    assert capi.validate(capi.Bsr(64, 64, 32, 32, dup.indptr, dup.indices)) == capi.BSP_OK
    assert capi.validate(_bsr([0, 0, 0, 0, 0], [])) == capi.BSP_OK  # no blocks at all


@pytest.mark.parametrize("name,kw,status,msg", BAD, ids=[b[0] for b in BAD])
def test_validate_rejects_malformed(name, kw, status, msg):
    assert capi.validate(_bsr(**kw)) == status
    assert msg in capi.last_error()


@pytest.mark.parametrize("H,Wd,R,C", [(100, 128, 32, 32), (128, 100, 32, 32), (128, 128, 0, 32),
                                      (128, 128, 32, -32)])
def test_validate_rejects_bad_shapes(H, Wd, R, C):
    nbr = max(1, H // max(R, 1))
    b = capi.Bsr(H, Wd, R, C, np.zeros(nbr + 1, np.int32), np.zeros(0, np.int32))
    assert capi.validate(b) == capi.BSP_ERR_BAD_STRUCTURE


def test_null_arguments():
    lib = capi.load()
    assert lib.bsp_validate_bsr(None) == capi.BSP_ERR_INVALID_ARGUMENT
    d = _bsr(**GOOD).desc()
    d.indptr = ctypes.cast(None, ctypes.POINTER(ctypes.c_int32))
    assert lib.bsp_validate_bsr(ctypes.byref(d)) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_spmm_plan_create(None, ctypes.byref(_bsr(**GOOD).desc()), 64, 0, 0, 0) == \
        capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_spmm(None, None, None, 0, None, 0, None) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_sddmm(None, None, None, 0, None, 0, None, None) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_attention_plan_create(None, ctypes.byref(_bsr(**GOOD).desc()), 64, 0, 0) == \
        capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_attention(None, None, None, 64, None, 64, None, 64, None, 64, None) == \
        capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_spgemm_plan_create(None, ctypes.byref(_bsr(**GOOD).desc()), ctypes.byref(_bsr(**GOOD).desc()),
                                      0, 0) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_spgemm(None, None, None, None, None) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_spgemm_structure(None, None, None, None) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_spgemm_symbolic(ctypes.byref(_bsr(**GOOD).desc()), ctypes.byref(_bsr(**GOOD).desc()), None,
                                   None, None) == capi.BSP_ERR_INVALID_ARGUMENT
    assert lib.bsp_plan_destroy(None) == capi.BSP_OK
    g = _bsr(**GOOD)
    assert lib.bsp_host_spmm(ctypes.byref(g.desc()), None, None, 64, None, 0, 0) == \
        capi.BSP_ERR_INVALID_ARGUMENT


def test_plan_create_rejects_before_touching_a_device():
    """Argument and structure errors are reported the same with or without a GPU."""
    lib = capi.load()
    h = ctypes.c_void_p()
    good = _bsr(**GOOD)
    assert lib.bsp_spmm_plan_create(ctypes.byref(h), ctypes.byref(good.desc()), 64, 0, 7, 0) == \
        capi.BSP_ERR_INVALID_ARGUMENT  # bad dtype
    assert lib.bsp_spmm_plan_create(ctypes.byref(h), ctypes.byref(good.desc()), 64, 5, 0, 0) == \
        capi.BSP_ERR_INVALID_ARGUMENT  # bad layout
    assert lib.bsp_spmm_plan_create(ctypes.byref(h), ctypes.byref(good.desc()), 64, 1, 0, 0) == \
        capi.BSP_ERR_UNSUPPORTED  # column-major B
    bad = _bsr(**BAD[0][1])
    assert lib.bsp_spmm_plan_create(ctypes.byref(h), ctypes.byref(bad.desc()), 64, 0, 0, 0) == \
        capi.BSP_ERR_BAD_STRUCTURE
    assert lib.bsp_sddmm_plan_create(ctypes.byref(h), ctypes.byref(bad.desc()), 64, 0, 0, 0) == \
        capi.BSP_ERR_BAD_STRUCTURE
    for d in (0, 48, 96, 256):  # the fused attention kernel takes head dimensions 32, 64, 128
        assert lib.bsp_attention_plan_create(ctypes.byref(h), ctypes.byref(good.desc()), d, 0, 0) == \
            capi.BSP_ERR_UNSUPPORTED
    assert lib.bsp_attention_plan_create(ctypes.byref(h), ctypes.byref(good.desc()), 64, 9, 0) == \
        capi.BSP_ERR_INVALID_ARGUMENT  # bad dtype
    assert lib.bsp_attention_plan_create(ctypes.byref(h), ctypes.byref(bad.desc()), 64, 0, 0) == \
        capi.BSP_ERR_BAD_STRUCTURE
    assert not h


def test_schedule_rejects_unsupported_sizes():
    odd = capi.Bsr(96, 96, 48, 48, np.array([0, 1, 1], np.int32), np.array([0], np.int32))
    with pytest.raises(capi.BsparseError) as e:
        capi.spmm_schedule(odd, 64)
    assert e.value.status == capi.BSP_ERR_UNSUPPORTED
    with pytest.raises(capi.BsparseError) as e:
        capi.spmm_schedule(_bsr(**GOOD), 48)  # N not a multiple of 32
    assert e.value.status == capi.BSP_ERR_UNSUPPORTED
    with pytest.raises(capi.BsparseError) as e:
        capi.sddmm_schedule(_bsr(**GOOD), 40)
    assert e.value.status == capi.BSP_ERR_UNSUPPORTED


# ---------------------------------------------------------------------------
# Schedule invariants
def _expected_entries(s):
    """{sub_row: [(b_row, a_off), ...]} in CSR order."""
    RS, CS = s.R // 32, s.C // 32
    exp = {}
    for sr in range(s.H // 32):
        i, sub = divmod(sr, RS)
        lst = []
        for blk in range(s.indptr[i], s.indptr[i + 1]):
            for t in range(CS):
                lst.append((int(s.indices[blk]) * s.C + 32 * t, blk * s.R * s.C + 32 * sub * s.C + 32 * t))
        exp[sr] = lst
    return exp


def _check_spmm_schedule(s, N, num_cus, split_env=None, monkeypatch=None):
    if split_env is not None:
        monkeypatch.setenv("BSP_SPMM_SPLIT", str(split_env))
    sch = capi.spmm_schedule(capi.Bsr(s.H, s.W, s.R, s.C, s.indptr, s.indices), N, num_cus)
    info, items = sch["info"], sch["items"]
    assert info["tile_n"] in (128, 256) and info["n_tiles"] == -(-N // info["tile_n"])
    exp = _expected_entries(s)
    seen = {sr: [] for sr in exp}
    slots = set()
    for row, e0, e1, slot, base, npieces in items:
        seen[row].append((e0, e1, slot, base, npieces))
    for sr, pieces in seen.items():
        assert pieces, f"sub-row {sr} has no work item (its output would not be written)"
        pieces.sort()
        ents = []
        for e0, e1, *_ in pieces:
            ents += list(zip(sch["ent_row"][e0:e1].tolist(), sch["ent_off"][e0:e1].tolist()))
        assert ents == exp[sr], f"sub-row {sr} entries differ"
        assert all(pieces[k][1] == pieces[k + 1][0] for k in range(len(pieces) - 1)), "pieces not contiguous"
        if len(pieces) == 1:
            assert pieces[0][2] == -1 and pieces[0][4] == 0
        else:
            base, npieces = pieces[0][3], pieces[0][4]
            assert npieces == len(pieces)
            assert sorted(p[2] for p in pieces) == list(range(base, base + npieces))
            assert all(p[3] == base and p[4] == npieces for p in pieces)
            slots.update(p[2] for p in pieces)
    assert len(slots) == info["n_slots"]
    assert info["max_item_entries"] == max((e1 - e0) for _, e0, e1, *_ in items)
    wg = sch["wgmap"]
    assert info["grid"] == wg.size and wg.size % 8 == 0
    real = np.sort(wg[wg >= 0])
    np.testing.assert_array_equal(real, np.arange(len(items) * info["n_tiles"]))
    # Each XCD (workgroup id modulo 8) covers whole column groups of its items.
    per_xcd = {}
    for g, u in enumerate(wg):
        if u >= 0:
            per_xcd.setdefault(g % 8, set()).add(u % info["n_tiles"])
    sizes = {len(t) for t in per_xcd.values()}
    assert len(sizes) <= 1, "XCDs cover unequal numbers of tiles"
    return sch


@pytest.mark.parametrize("num_cus", [8, 80, 256])
def test_spmm_schedule_uniform(num_cus):
    w = W.spmm_workload(2048, 2048, 512, 32, 32, 0.1, seed=1)
    _check_spmm_schedule(w["a"], 512, num_cus)


def test_spmm_schedule_skewed_splits_long_rows():
    """Rows longer than one compute unit's fair share are cut: the skewed
    structure planned for 1024 compute units (fair share 41 entries, its
    longest rows 101)."""
    s = W.workload_spmm_skewed()["a"]
    sch = _check_spmm_schedule(s, 1024, 1024)
    info = sch["info"]
    counts = np.diff(s.indptr)
    assert info["n_split_rows"] > 0
    assert info["max_item_entries"] < counts.max()
    # Per-XCD cost spread stays within one item's cost.
    costs = {}
    for g, u in enumerate(sch["wgmap"]):
        if u >= 0:
            it = sch["items"][u // info["n_tiles"]]
            costs[g % 8] = costs.get(g % 8, 0) + (it[2] - it[1]) + (4 if it[3] >= 0 else 2)
    assert max(costs.values()) - min(costs.values()) <= info["max_item_entries"] + 4


@pytest.mark.parametrize("split", [1, 2, 5])
def test_spmm_schedule_forced_splits(monkeypatch, split):
    w = W.spmm_workload(1024, 1024, 256, 32, 32, 0.3, seed=2)
    sch = _check_spmm_schedule(w["a"], 256, 256, split, monkeypatch)
    assert sch["info"]["max_item_entries"] <= split


@pytest.mark.parametrize("name,s", [
    ("R64", W.random_positions(512, 512, 64, 64, 20, np.random.default_rng(3))),
    ("R32C64", W.random_positions(512, 512, 32, 64, 30, np.random.default_rng(4))),
    ("R256", W.fill_tril(1024, 1024, 256, 256)),
    ("dups", W.fill_col_as_reference(128, 128, 32, 32, 10)),
    ("empty", W.BsrArrays(256, 256, 32, 32, np.zeros(9, np.int32), np.zeros(0, np.int32))),
])
def test_spmm_schedule_structures(name, s):
    _check_spmm_schedule(s, 128, 256)


def test_sddmm_schedule_covers_every_output_sub_block_once():
    rng = np.random.default_rng(8)
    for R, C in [(32, 32), (64, 32), (32, 64), (128, 128)]:
        m = W.random_positions(1024, 1024, R, C, 12, rng)
        sch = capi.sddmm_schedule(capi.Bsr(1024, 1024, R, C, m.indptr, m.indices), 64)
        offs = sorted(sch["ent_off"].tolist())
        expect = sorted(blk * R * C + 32 * s * C + 32 * t for blk in range(m.nblocks)
                        for s in range(R // 32) for t in range(C // 32))
        assert offs == expect
        covered = []
        for x_row0, e0, e1, *_ in sch["items"]:
            assert 0 < e1 - e0 <= sch["info"]["max_item_entries"]
            covered += list(range(e0, e1))
            for e in range(e0, e1):  # x rows of the item are the block row of its entries
                blk = sch["ent_off"][e] // (R * C)
                i = int(np.searchsorted(m.indptr, blk, side="right") - 1)
                assert i * R <= x_row0 < (i + 1) * R
        assert sorted(covered) == list(range(len(offs)))
        wg = sch["wgmap"]
        np.testing.assert_array_equal(np.sort(wg[wg >= 0]), np.arange(len(sch["items"])))


def test_sddmm_schedule_uniform_mask_two_column_bands_one_round():
    """The 4096^2 10% mask at K=256: stripes balanced by item count over four
    row groups let each XCD take one half of the mask's columns (half of Y)
    with every item still in one round of two workgroups per compute unit."""
    m = W.workload_sddmm()["mask"]
    sch = capi.sddmm_schedule(capi.Bsr(m.H, m.W, m.R, m.C, m.indptr, m.indices), 256, 256)
    assert sch["info"]["grid"] <= 2 * 256
    wg, items, cols = sch["wgmap"], sch["items"], sch["ent_row"]
    for x in range(8):
        us = wg[x::8]
        halves = {int(cols[e]) * 2 // m.W for u in us[us >= 0] for e in range(items[u][1], items[u][2])}
        assert len(halves) == 1, f"XCD {x} reads both column halves"


@pytest.mark.parametrize("group,R,C", [(2, 64, 64), (4, 128, 32), (8, 256, 256), (2, 128, 64)])
@pytest.mark.parametrize("split", [None, 2])
def test_spmm_schedule_row_groups(monkeypatch, group, R, C, split):
    """Group items cover every (stripe, sub-block product) exactly once: an
    item's entries serve stripes row..row+group-1 of one block row, and split
    groups give each stripe its own slots."""
    monkeypatch.setenv("BSP_SPMM_GROUP", str(group))
    if split:
        monkeypatch.setenv("BSP_SPMM_SPLIT", str(split))
    rng = np.random.default_rng(group * 7 + R)
    H = Wd = 2048
    m = W.random_positions(H, Wd, R, C, (H // R) * (Wd // C) // 3, rng)
    sch = capi.spmm_schedule(capi.Bsr(H, Wd, R, C, m.indptr, m.indices), 256)
    info = sch["info"]
    assert info["group"] == group and info["tile_n"] == 128
    RS, CS = R // 32, C // 32
    seen = []
    slots = set()
    for row, e0, e1, slot, base, npieces in sch["items"][:info["n_items"]]:
        assert row % group == 0
        i = (row * 32) // R
        for e in range(e0, e1):
            off = int(sch["ent_off"][e])
            blk, rem = divmod(off, R * C)
            assert m.indptr[i] <= blk < m.indptr[i + 1]
            t = (rem % C) // 32
            assert rem == (row % RS) * 32 * C + 32 * t
            assert sch["ent_row"][e] == m.indices[blk] * C + 32 * t
            for st in range(group):
                seen.append((row + st, blk, t))
        if slot >= 0:
            for st in range(group):
                s_ = base + st * npieces + (slot - base)
                assert s_ not in slots
                slots.add(s_)
    expect = [(i * RS + s, blk, t) for i in range(H // R) for blk in range(m.indptr[i], m.indptr[i + 1])
              for s in range(RS) for t in range(CS)]
    assert sorted(seen) == sorted(expect)
    assert len(slots) == info["n_slots"]


# ---------------------------------------------------------------------------
# SpGEMM symbolic phase (structure of A * B), host only.
def _rand(H, Wd, R, C, nblocks, seed):
    s = W.random_positions(H, Wd, R, C, nblocks, np.random.default_rng(seed))
    return s, capi.Bsr(s.H, s.W, s.R, s.C, s.indptr, s.indices)


@pytest.mark.parametrize("R,C,BC,na,nb", [(32, 32, 32, 20, 20), (64, 32, 32, 9, 30), (32, 64, 96, 14, 7),
                                          (128, 64, 32, 3, 25), (32, 32, 32, 0, 10), (32, 32, 32, 40, 44)])
def test_spgemm_symbolic_matches_oracle_structure(R, C, BC, na, nb):
    from helpers import orc
    a, ab = _rand(8 * R, 8 * C, R, C, na, R + na)
    b, bb = _rand(8 * C, 6 * BC, C, BC, nb, BC + nb)
    a.data = np.zeros(a.nblocks * R * C, np.uint16)
    b.data = np.zeros(b.nblocks * C * BC, np.uint16)
    indptr, indices, _ = orc.spgemm(a.indptr, a.indices, a.data, a.H, R, C, b.indptr, b.indices, b.data, b.W, BC)
    st = capi.spgemm_symbolic(ab, bb)
    assert (st.H, st.W, st.R, st.C) == (a.H, b.W, R, BC)
    np.testing.assert_array_equal(st.indptr, indptr)
    np.testing.assert_array_equal(st.indices, indices)


def test_spgemm_symbolic_duplicates_and_empty():
    a = _bsr([0, 2, 2, 3, 3], [1, 1, 3])                 # duplicate column 1 in row 0
    b = _bsr([0, 0, 2, 2, 3], [3, 0, 2])
    st = capi.spgemm_symbolic(a, b)
    np.testing.assert_array_equal(st.indptr, [0, 2, 2, 3, 3])
    np.testing.assert_array_equal(st.indices, [0, 3, 2])
    empty = _bsr([0, 0, 0, 0, 0], [])
    assert capi.spgemm_symbolic(empty, b).nblocks == 0
    assert capi.spgemm_symbolic(a, empty).nblocks == 0


def test_spgemm_rejects_mismatched_and_unsupported_operands():
    lib = capi.load()
    a = _bsr(**GOOD)
    n = ctypes.c_int64()
    cases = [
        (capi.Bsr(96, 128, 32, 32, np.zeros(4, np.int32), np.zeros(0, np.int32)), capi.BSP_ERR_INVALID_ARGUMENT,
         "rows"),                                                          # B.H != A.W
        (capi.Bsr(128, 128, 64, 32, np.zeros(3, np.int32), np.zeros(0, np.int32)), capi.BSP_ERR_INVALID_ARGUMENT,
         "block height"),                                                  # B.R != A.C
        (capi.Bsr(128, 96, 32, 48, np.zeros(5, np.int32), np.zeros(0, np.int32)), capi.BSP_ERR_UNSUPPORTED,
         "multiples of 32"),                                               # BC = 48
        (_bsr(**BAD[0][1]), capi.BSP_ERR_BAD_STRUCTURE, "B: indptr[0]"),
    ]
    for b, status, msg in cases:
        assert lib.bsp_spgemm_symbolic(ctypes.byref(a.desc()), ctypes.byref(b.desc()), ctypes.byref(n), None,
                                       None) == status
        assert msg in capi.last_error()
        h = ctypes.c_void_p()
        assert lib.bsp_spgemm_plan_create(ctypes.byref(h), ctypes.byref(a.desc()), ctypes.byref(b.desc()), 0,
                                          0) == status
        assert not h
    assert lib.bsp_spgemm_symbolic(ctypes.byref(_bsr(**BAD[1][1]).desc()), ctypes.byref(a.desc()),
                                   ctypes.byref(n), None, None) == capi.BSP_ERR_BAD_STRUCTURE
    assert capi.last_error().startswith("A: ")



@pytest.mark.gpu
def test_library_first_then_torch_shares_one_hip_runtime():
    """A process that creates a plan before torch touches the GPU must still
    find the GPU in torch: the binding loads torch's HIP runtime first, so
    the library binds to it (a second runtime would leave torch with none)."""
    import sys
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import __graft_entry__ as e\n"
        "capi = e.load_package().capi\n"
        "import numpy as np\n"
        "b = capi.Bsr(64, 64, 32, 32, np.array([0, 1, 2], np.int32), np.array([0, 1], np.int32))\n"
        "plan = capi.SpmmPlan(b, 64, 'f32')\n"
        "import torch\n"
        "x = torch.ones(4, device='cuda')\n"
        "torch.cuda.synchronize()\n"
        "print('ok', float(x.sum()))\n" % str(REPO))
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert p.returncode == 0 and "ok 4.0" in p.stdout, p.stdout[-2000:] + p.stderr[-2000:]


def test_noalloc_rejects_a_schedule_above_its_scratch_before_any_device_work():
    """bsp_spmm_noalloc checks its schedule against BSP_NOALLOC_SCRATCH_BYTES
    (and N against its tile) before it touches a device: 1M blocks times four
    128-column tiles need about 48 MB of entry words (24 MB at the widest
    tile)."""
    nbr = 1024
    indptr = np.arange(nbr + 1, dtype=np.int32) * 1024
    indices = np.tile(np.arange(1024, dtype=np.int32), nbr)
    d = capi.Bsr(nbr * 32, 1024 * 32, 32, 32, indptr, indices).desc()
    lib = capi.load()
    buf = ctypes.c_void_p(16)  # never dereferenced: the call fails before any device work
    st = lib.bsp_spmm_noalloc(ctypes.byref(d), buf, buf, 512, 512, buf, 512, capi.DTYPE_F32, 0, None)
    assert st == capi.BSP_ERR_UNSUPPORTED
    assert "no-allocation scratch" in capi.last_error()
    small = capi.Bsr(64, 64, 32, 32, np.array([0, 1, 1], np.int32), np.array([0], np.int32)).desc()
    st = lib.bsp_spmm_noalloc(ctypes.byref(small), buf, buf, 96, 96, buf, 96, capi.DTYPE_F32, 0, None)
    assert st == capi.BSP_ERR_UNSUPPORTED and "multiple of 128" in capi.last_error()
    assert capi.NOALLOC_SCRATCH_BYTES == 16 << 20


def test_noalloc_validates_the_structure_before_using_it():
    """A column index out of range or a null indptr is rejected as by
    bsp_validate_bsr, before the schedule builder reads the arrays (an
    out-of-range column would otherwise index host tables out of bounds)."""
    lib = capi.load()
    buf = ctypes.c_void_p(16)  # never dereferenced: the call fails before any device work
    nbr = 64
    indptr = np.arange(nbr + 1, dtype=np.int32) * 4
    indices = np.tile(np.array([0, 5, 9, 70], np.int32), nbr)  # 70 >= 64 block columns
    bsr = capi.Bsr(nbr * 32, 64 * 32, 32, 32, indptr, indices)
    d = bsr.desc()
    assert lib.bsp_validate_bsr(ctypes.byref(d)) == capi.BSP_ERR_BAD_STRUCTURE
    st = lib.bsp_spmm_noalloc(ctypes.byref(d), buf, buf, 4096, 4096, buf, 4096, capi.DTYPE_F32, 0, None)
    assert st == capi.BSP_ERR_BAD_STRUCTURE and "indices[" in capi.last_error()
    d.indptr = None
    st = lib.bsp_spmm_noalloc(ctypes.byref(d), buf, buf, 4096, 4096, buf, 4096, capi.DTYPE_F32, 0, None)
    assert st == capi.BSP_ERR_INVALID_ARGUMENT and "indptr is null" in capi.last_error()


def test_noalloc_reports_a_missing_device_as_an_error():
    """A valid call with no GPU visible returns BSP_ERR_DEVICE (never a
    silent default compute-unit count)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = capi.load()
    buf = ctypes.c_void_p(16)
    small = capi.Bsr(64, 64, 32, 32, np.array([0, 1, 1], np.int32), np.array([0], np.int32)).desc()
    st = lib.bsp_spmm_noalloc(ctypes.byref(small), buf, buf, 128, 128, buf, 128, capi.DTYPE_F32, 0, None)
    assert st == capi.BSP_ERR_DEVICE


class _OnGpu:
    """A CPU tensor presented as if it lived on cuda:`index` (the binding's
    operand checks read only these attributes), so that the checks run
    without a GPU."""

    def __init__(self, t, index=0):
        self._t, self._i = t, index
        self.is_cuda = True
        self.shape = t.shape

    @property
    def device(self):
        import torch
        return torch.device("cuda", self._i)

    def __getattr__(self, name):
        return getattr(self._t, name)


def test_binding_refuses_host_memory_and_mismatched_tensors():
    """The ctypes binding's run() operands: host arrays, CPU tensors, tensors on
    another GPU, wrong element size, a strided last dimension, a row stride
    that disagrees with ld, and a tensor too small for its operand are refused
    before anything reaches the library; a 2-D tensor's row stride becomes ld."""
    import torch
    op = capi._operand
    with pytest.raises(TypeError, match="numpy array is host memory"):
        op(np.zeros((4, 8), np.uint16), "b", 2, 4, 8, None, 0)
    with pytest.raises(ValueError, match="not on a GPU"):
        op(torch.zeros((4, 8), dtype=torch.int16), "b", 2, 4, 8, None, 0)
    with pytest.raises(ValueError, match="the plan on device 0"):
        op(_OnGpu(torch.zeros((4, 8), dtype=torch.int16), 1), "b", 2, 4, 8, None, 0)
    with pytest.raises(ValueError, match="elements of 4 bytes, expected 2"):
        op(_OnGpu(torch.zeros((4, 8), dtype=torch.float32)), "b", 2, 4, 8, None, 0)
    with pytest.raises(ValueError, match="last dimension must be contiguous"):
        op(_OnGpu(torch.zeros((8, 4), dtype=torch.int16).t()), "b", 2, 4, 8, None, 0)
    with pytest.raises(ValueError, match="row stride is 16"):
        op(_OnGpu(torch.zeros((4, 16), dtype=torch.int16)), "b", 2, 4, 8, 8, 0)
    with pytest.raises(ValueError, match="need 8"):
        op(_OnGpu(torch.zeros((4, 6), dtype=torch.int16)), "b", 2, 4, 8, None, 0)
    with pytest.raises(ValueError, match="covers 30 elements"):
        op(_OnGpu(torch.zeros(30, dtype=torch.int16)), "a_vals", 2, 1, 32, 32, 0)
    # a view that starts inside its storage: coverage counts from the view's start
    base = torch.zeros((5, 16), dtype=torch.int16)
    with pytest.raises(ValueError, match="covers"):
        op(_OnGpu(base[2:]), "b", 2, 4, 16, None, 0)
    # accepted: the row stride of a wider tensor becomes ld
    t = torch.zeros((4, 24), dtype=torch.int16)
    addr, ld = op(_OnGpu(t[:, :16]), "b", 2, 4, 16, None, 0)
    assert ld == 24 and addr == t.data_ptr()


def test_spmm_schedule_without_load_balancing(monkeypatch):
    """BSP_SPMM_BALANCE=0 (the reference's _no_lb operators): the skewed
    workload's rows stay whole, work items map to workgroups in natural
    order, and the products are still each scheduled once."""
    a = W.workload_spmm_skewed()["a"]
    bal = capi.spmm_schedule(bsr_of(a), 1024, 256)
    assert bal["info"]["n_split_rows"] >= 0
    monkeypatch.setenv("BSP_SPMM_BALANCE", "0")
    s = capi.spmm_schedule(bsr_of(a), 1024, 256)
    assert s["info"]["n_split_rows"] == 0
    assert np.array_equal(s["wgmap"], np.arange(len(s["wgmap"])))
    items = s["items"]
    assert np.all(items[:, 3] == -1)
    assert (items[:, 2] - items[:, 1]).sum() == a.nblocks
