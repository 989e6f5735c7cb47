"""Pins the oracle (oracle/bsp_oracle.c) on the CPU.

The reference commits no numeric golden vectors and its golden cannot be
compiled here (it includes tt-metal headers), so each oracle function is
pinned by what the mathematics fixes: the reference's own known-answer cases,
brute force in float64, invariants — and each check is shown to fail on a
planted mistake (the oracle's `mutation` argument).
"""
import numpy as np
import pytest

from helpers import W, orc

RNG = np.random.default_rng(1234)


def _rand_bsr(H, Wd, R, C, nblocks, seed):
    rng = np.random.default_rng(seed)
    s = W.random_positions(H, Wd, R, C, nblocks, rng)
    s.data = W.bf16_from_f32(W.uniform_f32(rng, s.nblocks * R * C))
    return s


def _spmm(s, b, mutation=0, threads=1):
    return orc.spmm(s.indptr, s.indices, s.data, s.H, s.W, s.R, s.C, b, threads=threads, mutation=mutation)


def _brute_spmm(s, b):
    """float64 sum over every stored block (duplicates included)."""
    bf = W.bf16_to_f32(b).astype(np.float64)
    out = np.zeros((s.H, b.shape[1]))
    vals = W.bf16_to_f32(s.data).astype(np.float64).reshape(-1, s.R, s.C)
    for i in range(s.nbrows):
        for blk in range(s.indptr[i], s.indptr[i + 1]):
            j = s.indices[blk]
            out[i * s.R:(i + 1) * s.R] += vals[blk] @ bf[j * s.C:(j + 1) * s.C]
    return out


def _brute_bound(s, b):
    """fp32 accumulation error bound: K_e * 2^-23 * sum |a||b| (generous)."""
    bf = np.abs(W.bf16_to_f32(b).astype(np.float64))
    absd = np.zeros((s.H, s.W))
    vals = np.abs(W.bf16_to_f32(s.data).astype(np.float64)).reshape(-1, s.R, s.C)
    for i in range(s.nbrows):
        for blk in range(s.indptr[i], s.indptr[i + 1]):
            j = s.indices[blk]
            absd[i * s.R:(i + 1) * s.R, j * s.C:(j + 1) * s.C] += vals[blk]
    kmax = max(1, int(np.diff(s.indptr).max(initial=0)) * s.C)
    return kmax * 2.0 ** -23 * (absd @ bf) + 1e-30


def _spmm_checks_pass(s, b, got) -> bool:
    return bool(np.all(np.abs(got - _brute_spmm(s, b)) <= _brute_bound(s, b)))


# ---------------------------------------------------------------------------
# bf16 conversion
def test_bf16_round_to_nearest_even_against_torch():
    import torch
    specials = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.01171875, 1.0078125, 3.0e38, -3.4e38,
                         1e-40, -1e-45, np.inf, -np.inf, 65504.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8],
                        dtype=np.float32)
    x = np.concatenate([specials, RNG.standard_normal(100000).astype(np.float32) * 1e3,
                        (RNG.random(10000).astype(np.float32) - 0.5) * 1e-38])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(orc.bf16_from_f32(x), ref)
    np.testing.assert_array_equal(W.bf16_from_f32(x), ref)
    nan = np.array([np.nan], np.float32)
    assert np.isnan(W.bf16_to_f32(orc.bf16_from_f32(nan)))[0]
    assert np.isnan(W.bf16_to_f32(W.bf16_from_f32(nan)))[0]
    np.testing.assert_array_equal(orc.bf16_to_f32(ref), W.bf16_to_f32(ref))


# ---------------------------------------------------------------------------
# SpMM golden: the reference's known answers (block_spmm/inc/test_suite.hpp:1862-1925)
def _one_block(content_a, content_b):
    s = W.fill_col(32, 32, 32, 32, 1)
    s.data = W.block_content(1, 32, 32, content_a)
    return s, W.dense_content(32, 32, content_b)


def test_spmm_1_block_id():
    s, b = _one_block("ID", "ID")
    np.testing.assert_array_equal(_spmm(s, b), np.eye(32, dtype=np.float32))


def test_spmm_1_block_uniform():
    s, b = _one_block("UNIFORM", "UNIFORM")
    np.testing.assert_array_equal(_spmm(s, b), np.full((32, 32), 32.0, np.float32))


def test_spmm_1_block_arange():
    s, b = _one_block("ARANGE", "UNIFORM")
    a = W.bf16_to_f32(s.data).reshape(32, 32).astype(np.float64)
    expect = np.repeat(a.sum(axis=1, keepdims=True), 32, axis=1)
    np.testing.assert_array_equal(_spmm(s, b), expect.astype(np.float32))


@pytest.mark.parametrize("R,C", [(32, 32), (64, 32), (32, 64), (64, 64)])
def test_spmm_brute_force(R, C):
    s = _rand_bsr(256, 384, R, C, 10, seed=R + C)
    b = W.bf16_from_f32(W.uniform_f32(np.random.default_rng(R * C), (384, 96)))
    assert _spmm_checks_pass(s, b, _spmm(s, b))


def test_spmm_duplicates_and_unsorted_columns_are_summed():
    s = W.fill_col_as_reference(64, 64, 32, 32, 4)  # rows [0,0] and [1,1]
    np.testing.assert_array_equal(s.indptr, [0, 2, 4])
    np.testing.assert_array_equal(s.indices, [0, 0, 1, 1])
    rng = np.random.default_rng(3)
    s.data = W.bf16_from_f32(W.uniform_f32(rng, 4 * 1024))
    b = W.bf16_from_f32(W.uniform_f32(rng, (64, 64)))
    assert _spmm_checks_pass(s, b, _spmm(s, b))
    u = W.BsrArrays(64, 96, 32, 32, np.array([0, 3, 3], np.int32), np.array([2, 0, 1], np.int32))
    u.data = W.bf16_from_f32(W.uniform_f32(rng, 3 * 1024))
    b2 = W.bf16_from_f32(W.uniform_f32(rng, (96, 64)))
    assert _spmm_checks_pass(u, b2, _spmm(u, b2))


def test_spmm_empty_rows_are_zero():
    s = W.BsrArrays(128, 128, 32, 32, np.array([0, 0, 1, 1, 1], np.int32), np.array([2], np.int32))
    s.data = W.bf16_from_f32(np.ones(1024, np.float32))
    out = _spmm(s, W.dense_content(128, 64, "UNIFORM"))
    assert np.all(out[:32] == 0) and np.all(out[64:] == 0) and np.all(out[32:64] == 32.0)


def test_spmm_threads_bit_identical():
    s = _rand_bsr(1024, 1024, 32, 32, 200, seed=5)
    b = W.bf16_from_f32(W.uniform_f32(np.random.default_rng(5), (1024, 128)))
    np.testing.assert_array_equal(_spmm(s, b, threads=1), _spmm(s, b, threads=4))


def test_spmm_matches_oracle_gemm_on_dense_expansion():
    """With distinct columns, SpMM == gemm_bfloat16(to_dense(A), B) to fp32 rounding."""
    s = _rand_bsr(128, 128, 32, 32, 6, seed=8)
    b = W.bf16_from_f32(W.uniform_f32(np.random.default_rng(8), (128, 64)))
    dense = orc.to_dense(s.indptr, s.indices, s.data, s.H, s.W, s.R, s.C)
    g = orc.gemm(dense, b)
    np.testing.assert_allclose(_spmm(s, b), g, rtol=0, atol=float(_brute_bound(s, b).max()) * 2)


@pytest.mark.parametrize("mutation", [1, 2, 3, 4])
def test_spmm_checks_catch_planted_mistakes(mutation):
    """Each plausible bug (1 transposed B, 2 dropped last block, 3 wrong sign,
    4 column index off by one) fails the brute-force check."""
    s = _rand_bsr(128, 128, 32, 32, 8, seed=11)
    b = W.bf16_from_f32(W.uniform_f32(np.random.default_rng(11), (128, 128)))
    assert _spmm_checks_pass(s, b, _spmm(s, b))
    assert not _spmm_checks_pass(s, b, _spmm(s, b, mutation=mutation))


def test_spmm_closed_forms_catch_planted_mistakes():
    s, b = _one_block("ARANGE", "UNIFORM")
    good = _spmm(s, b)
    for m in (2, 3):  # dropped block, wrong sign
        assert not np.array_equal(_spmm(s, b, mutation=m), good)


# ---------------------------------------------------------------------------
# SDDMM golden (sparse_common/bsr_matrix.hpp:816-857)
def _sddmm(m, x, y, mutation=0, colmajor=False):
    yy = np.ascontiguousarray(y.T) if colmajor else y
    return orc.sddmm(m.indptr, m.indices, m.data, m.H, m.W, m.R, m.C, x, yy, y_colmajor=colmajor,
                     mutation=mutation)


def _brute_sddmm(m, x, y):
    xf = W.bf16_to_f32(x).astype(np.float64)
    yf = W.bf16_to_f32(y).astype(np.float64)
    mv = W.bf16_to_f32(m.data).astype(np.float64).reshape(-1, m.R, m.C)
    out = np.empty_like(mv)
    ab = np.empty_like(mv)
    for i in range(m.nbrows):
        for blk in range(m.indptr[i], m.indptr[i + 1]):
            j = m.indices[blk]
            xs, ys = xf[i * m.R:(i + 1) * m.R], yf[:, j * m.C:(j + 1) * m.C]
            out[blk] = mv[blk] * (xs @ ys)
            ab[blk] = np.abs(mv[blk]) * (np.abs(xs) @ np.abs(ys))
    return out.ravel(), (x.shape[1] * 2.0 ** -23 * ab).ravel() + 1e-30


def _sddmm_checks_pass(m, x, y, got) -> bool:
    ref, bound = _brute_sddmm(m, x, y)
    return bool(np.all(np.abs(got - ref) <= bound))


def test_sddmm_uniform_arange_closed_form():
    """block_sddmm/inc/test_suite.hpp:27-110: out[r][c] = sum_k bf16(row*K + k)."""
    m = W.fill_row(64, 64, 32, 32, 4)
    m.data = W.block_content(4, 32, 32, "UNIFORM")
    x = W.dense_content(64, 64, "ARANGE")
    y = W.dense_content(64, 64, "UNIFORM")
    rows = W.bf16_to_f32(x).astype(np.float64).sum(axis=1)
    got = _sddmm(m, x, y).reshape(4, 32, 32)
    for blk, i in enumerate([0, 0, 1, 1]):
        np.testing.assert_array_equal(got[blk], np.repeat(rows[32 * i:32 * i + 32, None], 32, 1))


def test_sddmm_identity_mask_keeps_diagonals_only():
    m = W.fill_diag(128, 128, 32, 32, 4)
    m.data = W.block_content(4, 32, 32, "ID")
    rng = np.random.default_rng(2)
    x, y = W.dense_content(128, 64, "RAND", rng), W.dense_content(64, 128, "RAND", rng)
    got = _sddmm(m, x, y).reshape(4, 32, 32)
    assert np.all(got[:, ~np.eye(32, dtype=bool)] == 0)
    assert _sddmm_checks_pass(m, x, y, got.ravel())


def test_sddmm_full_mask_equals_dense_gemm_blocks():
    """test_full_mask (block_sddmm/inc/test_suite.hpp:45-52): every block
    present, mask 1.0 -> the blocks of gemm_bfloat16(X, Y) exactly (same
    k-order fp32 sums)."""
    m = W.fill_row(64, 96, 32, 32, 6)
    m.data = W.block_content(6, 32, 32, "UNIFORM")
    rng = np.random.default_rng(3)
    x, y = W.dense_content(64, 96, "RAND", rng), W.dense_content(96, 96, "RAND", rng)
    g = orc.gemm(x, y)
    got = _sddmm(m, x, y).reshape(6, 32, 32)
    for blk in range(6):
        i, j = divmod(blk, 3)
        np.testing.assert_array_equal(got[blk], g[32 * i:32 * i + 32, 32 * j:32 * j + 32])


@pytest.mark.parametrize("colmajor", [False, True])
@pytest.mark.parametrize("R,C", [(32, 32), (64, 32), (32, 64)])
def test_sddmm_brute_force(R, C, colmajor):
    rng = np.random.default_rng(R + 3 * C)
    m = W.random_positions(256, 256, R, C, 8, rng)
    m.data = W.bf16_from_f32(W.uniform_f32(rng, m.nblocks * R * C))
    x, y = W.dense_content(256, 96, "RAND", rng), W.dense_content(96, 256, "RAND", rng)
    assert _sddmm_checks_pass(m, x, y, _sddmm(m, x, y, colmajor=colmajor))


@pytest.mark.parametrize("mutation", [1, 2, 3, 4])
def test_sddmm_checks_catch_planted_mistakes(mutation):
    """1 mask values ignored, 2 Y transposed, 3 last k dropped, 4 wrong mask block."""
    rng = np.random.default_rng(17)
    m = W.random_positions(128, 128, 32, 32, 6, rng)
    m.data = W.bf16_from_f32(W.uniform_f32(rng, m.nblocks * 1024))
    x, y = W.dense_content(128, 128, "RAND", rng), W.dense_content(128, 128, "RAND", rng)
    assert _sddmm_checks_pass(m, x, y, _sddmm(m, x, y))
    assert not _sddmm_checks_pass(m, x, y, _sddmm(m, x, y, mutation=mutation))


# ---------------------------------------------------------------------------
def test_to_dense_small_case():
    s = W.BsrArrays(64, 96, 32, 32, np.array([0, 1, 2], np.int32), np.array([2, 0], np.int32))
    s.data = W.bf16_from_f32(np.concatenate([np.full(1024, 1.0), np.full(1024, 2.0)]).astype(np.float32))
    d = W.bf16_to_f32(orc.to_dense(s.indptr, s.indices, s.data, 64, 96, 32, 32))
    expect = np.zeros((64, 96), np.float32)
    expect[:32, 64:] = 1.0
    expect[32:, :32] = 2.0
    np.testing.assert_array_equal(d, expect)


def test_gemm_against_float64():
    rng = np.random.default_rng(9)
    a, b = W.dense_content(48, 200, "RAND", rng), W.dense_content(200, 40, "RAND", rng)
    af, bf = W.bf16_to_f32(a).astype(np.float64), W.bf16_to_f32(b).astype(np.float64)
    bound = 200 * 2.0 ** -23 * (np.abs(af) @ np.abs(bf))
    assert np.all(np.abs(orc.gemm(a, b) - af @ bf) <= bound)


def test_pcc_matches_numpy_and_limits():
    x = RNG.standard_normal(5000).astype(np.float32)
    y = (x + 0.3 * RNG.standard_normal(5000)).astype(np.float32)
    assert abs(orc.pcc(x, y) - np.corrcoef(x, y)[0, 1]) < 1e-4
    assert abs(orc.pcc(x, x) - 1.0) < 1e-5
    assert abs(orc.pcc(x, -x) + 1.0) < 1e-5


def test_small_vectors_fixture_reproduced():
    from golden_fixtures import small_vectors
    v = small_vectors()
    M, K, R, C = (int(t) for t in v["spmm_shape"])
    np.testing.assert_array_equal(
        orc.spmm(v["spmm_indptr"], v["spmm_indices"], v["spmm_a"], M, K, R, C, v["spmm_b"]), v["spmm_golden"])
    M, N, R, C = (int(t) for t in v["sddmm_shape"])
    np.testing.assert_array_equal(
        orc.sddmm(v["sddmm_indptr"], v["sddmm_indices"], v["sddmm_mask"], M, N, R, C, v["sddmm_x"],
                  v["sddmm_y"]), v["sddmm_golden"])


# ---------------------------------------------------------------------------
# SpGEMM golden (sparse_common/bsr_matrix.hpp:741-810): BSR x BSR -> BSR
def _spgemm(a, b, mutation=0):
    return orc.spgemm(a.indptr, a.indices, a.data, a.H, a.R, a.C, b.indptr, b.indices, b.data, b.W, b.C,
                      mutation=mutation)


def _pattern(s):
    p = np.zeros((s.H // s.R, s.W // s.C), np.int64)
    for i in range(s.nbrows):
        for blk in range(s.indptr[i], s.indptr[i + 1]):
            p[i, s.indices[blk]] += 1
    return p


def _brute_spgemm(a, b):
    """float64 dense product of every stored block (duplicates summed) and the
    fp32 accumulation bound of the golden: (pairs * C) * 2^-23 * |A||B|."""
    def dense(s):
        d = np.zeros((s.H, s.W))
        v = W.bf16_to_f32(s.data).astype(np.float64).reshape(-1, s.R, s.C)
        for i in range(s.nbrows):
            for blk in range(s.indptr[i], s.indptr[i + 1]):
                j = s.indices[blk]
                d[i * s.R:(i + 1) * s.R, j * s.C:(j + 1) * s.C] += v[blk]
        return d
    ad, bd = dense(a), dense(b)
    pairs = max(1, int((_pattern(a) @ _pattern(b)).max(initial=0)))
    return ad @ bd, pairs * a.C * 2.0 ** -23 * (np.abs(ad) @ np.abs(bd)) + 1e-30


def _spgemm_checks_pass(a, b, got) -> bool:
    """Structure equals the boolean product of the block patterns, columns
    ascending per row; every stored value within the bound of the float64
    product; every product entry outside the structure is zero."""
    indptr, indices, vals = got
    want = (_pattern(a) @ _pattern(b)) > 0
    nbr, nbc = want.shape
    R, BC = a.R, b.C
    if indptr.size != nbr + 1 or indptr[-1] != indices.size or vals.size != indices.size * R * BC:
        return False
    ref, bound = _brute_spgemm(a, b)
    covered = np.zeros((a.H, b.W), bool)
    for i in range(nbr):
        cols = indices[indptr[i]:indptr[i + 1]]
        if not np.array_equal(cols, np.flatnonzero(want[i])):
            return False
        for n, j in enumerate(cols):
            blk = vals[(indptr[i] + n) * R * BC:(indptr[i] + n + 1) * R * BC].reshape(R, BC).astype(np.float64)
            sl = (slice(i * R, (i + 1) * R), slice(j * BC, (j + 1) * BC))
            covered[sl] = True
            if not np.all(np.abs(blk - ref[sl]) <= bound[sl]):
                return False
    return bool(np.all(ref[~covered] == 0))


def test_spgemm_block_identity_returns_a():
    """B = block-diagonal identity: every output block is one A block times I,
    an exact product (one nonzero term per element)."""
    a = _rand_bsr(128, 192, 32, 32, 9, 41)
    b = W.fill_diag(192, 192, 32, 32, 6)
    b.data = W.block_content(6, 32, 32, "ID")
    indptr, indices, vals = _spgemm(a, b)
    np.testing.assert_array_equal(indptr, a.indptr)
    np.testing.assert_array_equal(indices, a.indices)
    np.testing.assert_array_equal(vals, W.bf16_to_f32(a.data))


def test_spgemm_uniform_closed_form():
    """All-ones blocks: output element = (pairs contributing) * C exactly."""
    a = W.fill_row(64, 128, 32, 32, 6)     # rows 0: cols 0..3, row 1: cols 0,1
    a.data = W.block_content(6, 32, 32, "UNIFORM")
    b = W.fill_diag(128, 128, 32, 32, 4)
    b.data = W.block_content(4, 32, 32, "UNIFORM")
    indptr, indices, vals = _spgemm(a, b)
    np.testing.assert_array_equal(indptr, [0, 4, 6])
    np.testing.assert_array_equal(indices, [0, 1, 2, 3, 0, 1])
    np.testing.assert_array_equal(vals, np.full(6 * 1024, 32.0, np.float32))


@pytest.mark.parametrize("R,C,BC", [(32, 32, 32), (64, 32, 32), (32, 64, 32), (32, 32, 64), (64, 64, 32)])
def test_spgemm_brute_force(R, C, BC):
    a = _rand_bsr(4 * R, 6 * C, R, C, 9, R + 7 * C)
    b = _rand_bsr(6 * C, 5 * BC, C, BC, 12, 3 * R + BC)
    assert _spgemm_checks_pass(a, b, _spgemm(a, b))


def test_spgemm_duplicates_and_empty_rows():
    """A duplicate (row, column) block contributes once per stored copy, as in
    the golden's loop; an empty block row of A gives an empty output row."""
    rng = np.random.default_rng(5)
    a = W.BsrArrays(128, 96, 32, 32, np.array([0, 3, 3, 4, 5], np.int32), np.array([2, 0, 2, 1, 1], np.int32))
    a.data = W.bf16_from_f32(W.uniform_f32(rng, 5 * 1024))
    b = _rand_bsr(96, 128, 32, 32, 5, 6)
    got = _spgemm(a, b)
    assert got[0][2] == got[0][1]
    assert _spgemm_checks_pass(a, b, got)


def test_spgemm_structure_from_pattern_not_values():
    """Zero-valued blocks still make output blocks (the golden marks presence
    from the structure alone, :763-766)."""
    a = W.fill_diag(64, 64, 32, 32, 2)
    a.data = np.zeros(2 * 1024, np.uint16)
    b = W.fill_row(64, 64, 32, 32, 4)
    b.data = W.block_content(4, 32, 32, "UNIFORM")
    indptr, indices, vals = _spgemm(a, b)
    np.testing.assert_array_equal(indptr, [0, 2, 4])
    np.testing.assert_array_equal(indices, [0, 1, 0, 1])
    assert np.all(vals == 0)


@pytest.mark.parametrize("mutation", [1, 2, 3, 4])
def test_spgemm_checks_catch_planted_mistakes(mutation):
    """1 B block transposed, 2 last A block of each row skipped, 3 output
    column shifted, 4 first c term dropped."""
    a = _rand_bsr(128, 128, 32, 32, 8, 21)
    b = _rand_bsr(128, 128, 32, 32, 8, 22)
    assert _spgemm_checks_pass(a, b, _spgemm(a, b))
    assert not _spgemm_checks_pass(a, b, _spgemm(a, b, mutation=mutation))
