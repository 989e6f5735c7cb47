"""Seeded synthetic inputs: the reference's structure generators and the five
benchmark workloads.

Structure generators restate the fill modes of bsr_matrix<T>'s constructors
(sparse_common/bsr_matrix.hpp:244-408, block_spmm/inc/bsr_matrix.hpp:376-405
for FILL_TRIU) and its random-position constructor (:619-679).  The reference
seeds positions from the clock and values from unseeded rand()
(sparse_common/bsr_matrix.hpp:646-647, :55).  Here every benchmark workload
comes from this module's own seeded generator (Rng: xoshiro256**, seeded
through splitmix64), written in plain uint64 arithmetic, so its output does
not depend on numpy's own generators (whose streams numpy does not promise to
keep across versions) and is identical on every machine; workload_digest()
pins each workload's bytes.  Values are drawn in float32 and rounded to bf16
(round to nearest even), returned as uint16 bit patterns.  The generator
functions also accept a numpy Generator (tests use them for inputs that are
checked against the oracle in the same run and need no pinning).
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Optional

import numpy as np

SEED_BASE = 0x5EED0000  # workload i uses SEED_BASE + i
TILE = 32

_M64 = (1 << 64) - 1


class Rng:
    """xoshiro256** (D. Blackman and S. Vigna, "Scrambled linear pseudorandom
    number generators", 2018), run as `lanes` independent streams stepped
    together: the state of lane l is four outputs of splitmix64 started at
    seed * lanes + l.  Output k of a draw is step k // lanes of lane
    k % lanes; a draw consumes whole steps.  uint64 arithmetic wraps, as the
    algorithm requires; nothing else (no float library call) enters the
    integer streams."""

    def __init__(self, seed: int, lanes: int = 65536):
        self.lanes = lanes
        x = (np.uint64(seed & _M64) * np.uint64(lanes) + np.arange(lanes, dtype=np.uint64))
        st = []
        with np.errstate(over="ignore"):
            for _ in range(4):
                x = x + np.uint64(0x9E3779B97F4A7C15)
                z = x.copy()
                z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
                z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
                st.append(z ^ (z >> np.uint64(31)))
        self.s = st

    @staticmethod
    def _rotl(x, k):
        return (x << np.uint64(k)) | (x >> np.uint64(64 - k))

    def u64(self, n: int) -> np.ndarray:
        """n uint64 outputs."""
        steps = -(-n // self.lanes)
        out = np.empty((max(steps, 0), self.lanes), np.uint64)
        s0, s1, s2, s3 = self.s
        with np.errstate(over="ignore"):
            for i in range(steps):
                out[i] = self._rotl(s1 * np.uint64(5), 7) * np.uint64(9)
                t = s1 << np.uint64(17)
                s2 = s2 ^ s0
                s3 = s3 ^ s1
                s1 = s1 ^ s2
                s0 = s0 ^ s3
                s2 = s2 ^ t
                s3 = self._rotl(s3, 45)
        self.s = [s0, s1, s2, s3]
        return out.reshape(-1)[:n]

    def random(self, shape, dtype=np.float64) -> np.ndarray:
        """U[0, 1): float64 from the top 53 bits, float32 from the top 24
        (both exact)."""
        n = int(np.prod(shape))
        x = self.u64(n)
        if np.dtype(dtype) == np.float32:
            r = (x >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
        else:
            r = (x >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        return r.reshape(shape)

    def standard_normal(self, shape, dtype=np.float32) -> np.ndarray:
        """N(0, 1) by the Box-Muller transform of two float64 uniforms."""
        n = int(np.prod(shape))
        u1 = 1.0 - self.random(n)  # (0, 1]
        u2 = self.random(n)
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return z.astype(dtype).reshape(shape)

    def sample(self, n: int, k: int) -> np.ndarray:
        """k distinct integers of [0, n), ascending: the k smallest of n random
        keys (a uniform k-subset; ties broken by position)."""
        keys = self.u64(n)
        return np.sort(np.argsort(keys, kind="stable")[:k]).astype(np.int64)


def _sample_sorted(rng, n: int, k: int) -> np.ndarray:
    if isinstance(rng, Rng):
        return rng.sample(n, k)
    return np.sort(rng.choice(n, size=k, replace=False)).astype(np.int64)


def workload_digest(w: dict) -> str:
    """SHA-256 over a workload's arrays (BSR index arrays and values, dense
    operands) in key order, with each array's dtype and shape."""
    h = hashlib.sha256()
    for key in sorted(w):
        v = w[key]
        parts = []
        if isinstance(v, BsrArrays):
            parts = [("indptr", v.indptr), ("indices", v.indices), ("data", v.data)]
        elif isinstance(v, np.ndarray):
            parts = [("", v)]
        for name, arr in parts:
            if arr is None:
                continue
            arr = np.ascontiguousarray(arr)
            h.update(f"{key}.{name}:{arr.dtype.str}:{arr.shape}".encode())
            h.update(arr.tobytes())
    return h.hexdigest()


# ---------------------------------------------------------------------------
# bf16
def bf16_from_f32(x) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN kept quiet)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32)
    # uint32 arithmetic wraps only for NaN patterns, which are replaced below.
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r.reshape(f.shape)


def uniform_f32(rng: np.random.Generator, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """float32 U[lo, hi) from the generator's float32 stream."""
    x = rng.random(shape, dtype=np.float32)
    np.multiply(x, np.float32(hi - lo), out=x)
    np.add(x, np.float32(lo), out=x)
    return x


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32).reshape(h.shape)


# ---------------------------------------------------------------------------
@dataclass
class BsrArrays:
    """A BSR matrix with bf16 block values (bsr_matrix<bfloat16>)."""

    H: int
    W: int
    R: int
    C: int
    indptr: np.ndarray   # int32 [H/R + 1]
    indices: np.ndarray  # int32 [nblocks]
    data: Optional[np.ndarray] = None  # uint16 [nblocks * R * C]

    @property
    def nblocks(self) -> int:
        return int(self.indices.size)

    @property
    def nbrows(self) -> int:
        return self.H // self.R

    @property
    def nbcols(self) -> int:
        return self.W // self.C

    def block_rows(self) -> np.ndarray:
        """Block-row index of every stored block."""
        return np.repeat(np.arange(self.nbrows, dtype=np.int32), np.diff(self.indptr))


def _from_positions(H, W, R, C, rows, cols) -> BsrArrays:
    """CSR arrays from block positions, kept in the given order within a row
    (a stable sort by row only)."""
    rows = np.asarray(rows, dtype=np.int64)
    cols = np.asarray(cols, dtype=np.int64)
    order = np.argsort(rows, kind="stable")
    rows, cols = rows[order], cols[order]
    nbr = H // R
    counts = np.bincount(rows, minlength=nbr) if rows.size else np.zeros(nbr, np.int64)
    indptr = np.zeros(nbr + 1, np.int32)
    np.cumsum(counts, out=indptr[1:])
    return BsrArrays(H, W, R, C, indptr, cols.astype(np.int32))


# Fill modes of sparse_common/bsr_matrix.hpp:17-21 and block_spmm's FILL_TRIU.
def fill_row(H, W, R, C, nblocks) -> BsrArrays:
    """FILL_ROW (:264-290): the first nblocks block positions in row-major order."""
    nbc = W // C
    flat = np.arange(min(nblocks, (H // R) * nbc))
    return _from_positions(H, W, R, C, flat // nbc, flat % nbc)


def fill_col(H, W, R, C, nblocks) -> BsrArrays:
    """Column fill: the first nblocks block positions in column-major order,
    stored as a valid CSR matrix (sorted columns per row).  The reference's
    FILL_COL (:291-317) writes indices in column-major order against row
    counts; see fill_col_as_reference for that structure."""
    nbr = H // R
    flat = np.arange(min(nblocks, nbr * (W // C)))
    return _from_positions(H, W, R, C, flat % nbr, flat // nbr)


def fill_col_as_reference(H, W, R, C, nblocks) -> BsrArrays:
    """The exact index arrays the reference's content-typed FILL_COL loop
    produces (sparse_common/bsr_matrix.hpp:291-317): rows counted per block
    row but indices pushed in column-major visiting order, which yields
    duplicate and misplaced columns once nblocks > H/R.  Used to show that the
    kernels accept such structures and sum duplicates as the golden does."""
    nbr, nbc = H // R, W // C
    indptr = np.zeros(nbr + 1, np.int64)
    indices = []
    for j in range(nbc):
        for i in range(nbr):
            if i + j * nbr < nblocks:
                indptr[i + 1] += 1
                indices.append(j)
    indptr = np.cumsum(indptr).astype(np.int32)
    return BsrArrays(H, W, R, C, indptr, np.asarray(indices, np.int32))


def fill_diag(H, W, R, C, nblocks) -> BsrArrays:
    """FILL_DIAG (:318-343): blocks (i, i) for i < nblocks."""
    assert nblocks <= min(H // R, W // C)
    i = np.arange(nblocks)
    return _from_positions(H, W, R, C, i, i)


def fill_tril(H, W, R, C) -> BsrArrays:
    """FILL_TRIL (:344-372): all blocks with j <= i (square block grid)."""
    n = H // R
    assert n == W // C
    r, c = np.tril_indices(n)
    return _from_positions(H, W, R, C, r, c)


def fill_triu(H, W, R, C) -> BsrArrays:
    """FILL_TRIU (block_spmm/inc/bsr_matrix.hpp, the SpMM-side copy): j >= i."""
    n = H // R
    assert n == W // C
    r, c = np.triu_indices(n)
    return _from_positions(H, W, R, C, r, c)


def multi_diag_positions(nbr: int, nbc: int, nblocks: int):
    """bsr_matrix::multi_diag_positions (sparse_common/bsr_matrix.hpp:215-240):
    diagonals d = 0, +1, -1, +2, -2, ... filled until nblocks positions, then
    sorted."""
    pos = []
    d = 0
    while len(pos) < nblocks:
        if d >= 0:
            i = 0
            while i < nbr and i + d < nbc and len(pos) < nblocks:
                pos.append((i, i + d))
                i += 1
        else:
            ad = -d
            j = 0
            while j < nbc and j + ad < nbr and len(pos) < nblocks:
                pos.append((j + ad, j))
                j += 1
        d = -d + 1 if d <= 0 else -d
        if abs(d) >= max(nbr, nbc):
            break
    pos.sort()
    return pos


def fill_multi_diag(H, W, R, C, nblocks) -> BsrArrays:
    pos = multi_diag_positions(H // R, W // C, nblocks)
    r = [p[0] for p in pos]
    c = [p[1] for p in pos]
    return _from_positions(H, W, R, C, r, c)


def random_positions(H, W, R, C, nblocks, rng: np.random.Generator) -> BsrArrays:
    """Uniform-random distinct block positions (the random-position
    constructor, sparse_common/bsr_matrix.hpp:619-679, with a seeded
    generator), columns sorted within each row."""
    nbr, nbc = H // R, W // C
    flat = _sample_sorted(rng, nbr * nbc, nblocks)
    return _from_positions(H, W, R, C, flat // nbc, flat % nbc)


# Content types of sparse_common/bsr_matrix.hpp:28-33.
def block_content(nblocks: int, R: int, C: int, content: str, rng: Optional[np.random.Generator] = None):
    """Block values as the reference fills them per block: RAND (here U[-1,1]),
    UNIFORM (1.0), ID (1 on r == c), ARANGE (r*C + c within each block)."""
    n = nblocks * R * C
    if content == "RAND":
        return bf16_from_f32(uniform_f32(rng, n))
    k = np.tile(np.arange(R * C), nblocks)
    if content == "UNIFORM":
        return bf16_from_f32(np.ones(n, np.float32))
    if content == "ID":
        return bf16_from_f32(((k // C) == (k % C)).astype(np.float32))
    if content == "ARANGE":
        return bf16_from_f32(k.astype(np.float32))
    raise ValueError(content)


def dense_content(H: int, W: int, content: str, rng: Optional[np.random.Generator] = None):
    """dense_matrix(rows, cols, content) (sparse_common/bsr_matrix.hpp:48-79):
    RAND (here U[-1,1]), UNIFORM, ID (i == j), ARANGE (flat index)."""
    if content == "RAND":
        return bf16_from_f32(uniform_f32(rng, (H, W)))
    k = np.arange(H * W).reshape(H, W)
    if content == "UNIFORM":
        return bf16_from_f32(np.ones((H, W), np.float32))
    if content == "ID":
        return bf16_from_f32(((k // W) == (k % W)).astype(np.float32))
    if content == "ARANGE":
        return bf16_from_f32(k.astype(np.float32))
    raise ValueError(content)


# ---------------------------------------------------------------------------
# Benchmark workloads.
def zipf_row_counts(nbr: int, nbc: int, density: float, s: float, cap: int,
                    rng: np.random.Generator) -> np.ndarray:
    """Per-row block counts: Zipf(s) on {1..cap} by inverse CDF, rescaled to a
    total of round(density * nbr * nbc) with largest-remainder rounding, no
    row above cap."""
    k = np.arange(1, cap + 1, dtype=np.float64)
    pmf = k ** (-s)
    cdf = np.cumsum(pmf / pmf.sum())
    u = rng.random(nbr)
    raw = np.minimum(np.searchsorted(cdf, u, side="left") + 1, cap).astype(np.float64)
    cap = min(cap, nbc)
    target = min(int(round(density * nbr * nbc)), nbr * cap)
    capped = np.zeros(nbr, bool)
    while True:
        remaining = target - cap * int(capped.sum())
        w = np.where(capped, 0.0, raw)
        scaled = w * remaining / w.sum()
        base = np.floor(scaled).astype(np.int64)
        short = remaining - int(base.sum())
        frac = np.where(capped, -1.0, scaled - base)
        order = np.lexsort((np.arange(nbr), -frac))  # largest remainder, ties by row
        base[order[:short]] += 1
        counts = np.where(capped, cap, base)
        over = counts > cap
        if not over.any():
            return counts.astype(np.int64)
        capped |= over  # pin the overflowing rows at the cap and rescale the rest


def spmm_workload(M, K, N, R, C, density: float, seed: int, value_range=1.0, zipf=None) -> dict:
    """A (BSR, random positions or Zipf rows) and B dense, both bf16
    U[-value_range, value_range]."""
    rng = Rng(seed)
    nbr, nbc = M // R, K // C
    if zipf is None:
        nnzb = int(round(density * nbr * nbc))
        a = random_positions(M, K, R, C, nnzb, rng)
    else:
        s, cap = zipf
        counts = zipf_row_counts(nbr, nbc, density, s, cap, rng)
        # Row i's columns: the cnt smallest of its nbc random keys (a uniform
        # subset per row, as _sample_sorted draws one).
        keys = rng.u64(nbr * nbc).reshape(nbr, nbc) if isinstance(rng, Rng) else None
        rows, cols = [], []
        for i, cnt in enumerate(counts):
            if cnt:
                if keys is not None:
                    cs = np.sort(np.argsort(keys[i], kind="stable")[: int(cnt)]).astype(np.int64)
                else:
                    cs = _sample_sorted(rng, nbc, int(cnt))
                rows.append(np.full(cnt, i))
                cols.append(cs)
        a = _from_positions(M, K, R, C, np.concatenate(rows), np.concatenate(cols))
    a.data = bf16_from_f32(uniform_f32(rng, a.nblocks * R * C, -value_range, value_range))
    b = bf16_from_f32(uniform_f32(rng, (K, N), -value_range, value_range))
    return {"a": a, "b": b, "M": M, "K": K, "N": N}


SPMM_SWEEP_DENSITIES = (0.01, 0.05, 0.25, 0.50)


def workload_spmm_large_blocks(density=0.25, R=256, seed=SEED_BASE + 5) -> dict:
    """The reference's published SpMM configuration (M = N = K = 8192,
    256 x 256 blocks, uniform-random positions;
    block_spmm/scripts/experiments_dram_reads_table.tex:27-35): A and B bf16
    U[-1, 1]."""
    return spmm_workload(8192, 8192, 8192, R, R, density, seed)


def workload_spmm_small() -> dict:
    """A 1024x1024, 32x32 blocks, 10% uniform positions, B 1024x256, U[-1,1]."""
    return spmm_workload(1024, 1024, 256, 32, 32, 0.10, SEED_BASE + 0)


def workload_spmm_sweep(density: float) -> dict:
    """A 4096x4096, 32x32 blocks at `density`, B 4096x512, U[-1,1]."""
    idx = {0.01: 0, 0.05: 1, 0.25: 2, 0.50: 3}.get(density, 9)
    return spmm_workload(4096, 4096, 512, 32, 32, density, SEED_BASE + 1 + 16 * idx)


def workload_sddmm(M=4096, N=4096, K=256, density=0.10, seed=SEED_BASE + 2) -> dict:
    """mask M x N (32x32 blocks, uniform positions, values 1.0), X M x K and
    Y K x N, both N(0,1) bf16."""
    rng = Rng(seed)
    nnzb = int(round(density * (M // 32) * (N // 32)))
    mask = random_positions(M, N, 32, 32, nnzb, rng)
    mask.data = bf16_from_f32(np.ones(nnzb * 1024, np.float32))
    x = bf16_from_f32(rng.standard_normal((M, K), dtype=np.float32))
    y = bf16_from_f32(rng.standard_normal((K, N), dtype=np.float32))
    return {"mask": mask, "x": x, "y": y, "M": M, "N": N, "K": K}


def workload_spgemm(n=8192, block=32, density=0.05, seed=SEED_BASE + 6) -> dict:
    """A and B n x n, block x block blocks at uniform-random positions with
    `density` each, values U[-1, 1] bf16 (A * B with 32x32 blocks at 5%: about
    47% of the output blocks are stored, 0.64 block pairs each on average)."""
    rng = Rng(seed)
    nnzb = int(round(density * (n // block) ** 2))
    a = random_positions(n, n, block, block, nnzb, rng)
    a.data = bf16_from_f32(uniform_f32(rng, nnzb * block * block))
    b = random_positions(n, n, block, block, nnzb, rng)
    b.data = bf16_from_f32(uniform_f32(rng, nnzb * block * block))
    return {"a": a, "b": b, "n": n, "block": block, "density": density}


def workload_spmm_skewed() -> dict:
    """A 16384x16384, 32x32 blocks, Zipf(1.2) rows capped at 512, 2% mean
    density; B 16384x1024; U[-1,1]."""
    return spmm_workload(16384, 16384, 1024, 32, 32, 0.02, SEED_BASE + 3, zipf=(1.2, 512))


def band_global_mask(seq: int, block: int, bands: int, global_density: float,
                     rng: np.random.Generator) -> BsrArrays:
    """Causal local window of `bands` block diagonals (offsets 0, -1, ..,
    -(bands-1)) plus uniform-random global blocks outside the band, numbering
    round(global_density * nb^2)."""
    nb = seq // block
    i, j = np.meshgrid(np.arange(nb), np.arange(nb), indexing="ij")
    band = (i - j >= 0) & (i - j < bands)
    outside = np.flatnonzero(~band.ravel())
    ng = int(round(global_density * nb * nb))
    pick = outside[_sample_sorted(rng, outside.size, ng)]
    flat = np.sort(np.concatenate([np.flatnonzero(band.ravel()), pick]))
    return _from_positions(seq, seq, block, block, flat // nb, flat % nb)


def workload_attention(seq=8192, d=128, seed=SEED_BASE + 4) -> dict:
    """Q, K, V seq x d, N(0, std = d^-1/2) bf16; mask = 8 causal block
    diagonals + 1% global blocks, values 1.0."""
    rng = Rng(seed)
    mask = band_global_mask(seq, 32, 8, 0.01, rng)
    mask.data = bf16_from_f32(np.ones(mask.nblocks * 1024, np.float32))
    std = d ** -0.5
    q = bf16_from_f32(rng.standard_normal((seq, d), dtype=np.float32) * np.float32(std))
    k = bf16_from_f32(rng.standard_normal((seq, d), dtype=np.float32) * np.float32(std))
    v = bf16_from_f32(rng.standard_normal((seq, d), dtype=np.float32) * np.float32(std))
    return {"mask": mask, "q": q, "k": k, "v": v, "seq": seq, "d": d}


# ---------------------------------------------------------------------------
# Algorithmic FLOP and byte counts (the reference's FLOP formulas,
# GEMM_profiling/read_spmm_profiler.py:73 and read_sddmm_profiler.py:75).
def spmm_flops(nblocks: int, R: int, C: int, N: int) -> float:
    return 2.0 * nblocks * R * C * N


def sddmm_flops(nblocks: int, R: int, C: int, K: int) -> float:
    return 2.0 * nblocks * R * C * K + nblocks * R * C


def spmm_bytes(a: BsrArrays, N: int, out_bytes: int) -> float:
    """A values + index arrays + the B panels touched (once each) + the whole
    dense output."""
    touched = np.unique(a.indices).size
    return (2.0 * a.nblocks * a.R * a.C + 4.0 * (a.nblocks + a.nbrows + 1)
            + 2.0 * a.C * N * touched + float(a.H) * N * out_bytes)


def sddmm_bytes(mask: BsrArrays, K: int, out_bytes: int, mask_values: bool = True) -> float:
    """X + Y + mask values + index arrays + output blocks."""
    blk = mask.nblocks * mask.R * mask.C
    return (2.0 * mask.H * K + 2.0 * K * mask.W + (2.0 * blk if mask_values else 0.0)
            + 4.0 * (mask.nblocks + mask.nbrows + 1) + float(blk) * out_bytes)
