"""The benchmark workloads are pinned: their bytes (structure, block values,
dense operands) hash to the SHA-256 digests below on every machine.  They
come from the package's own xoshiro256** generator (workloads.Rng), whose
integer streams are checked here against the generator's published recurrence
(splitmix64 seeding, then xoshiro256**) restated in Python integers."""
import numpy as np
import pytest

from helpers import W

# workload -> SHA-256 of workloads.workload_digest(...)
DIGESTS = {
    "C1 small 1024^2 10% N=256": ("workload_spmm_small", (),
                                  "6da301e1e252883ce4f3c0e8039635161ead00914372ded57d6371e7b91dd726"),
    "C2 4096^2 1% N=512": ("workload_spmm_sweep", (0.01,),
                           "1c790b20b031d760b2adb846e33890babc2e543a5faa23ab9d5e72cf7c75d671"),
    "C2 4096^2 5% N=512": ("workload_spmm_sweep", (0.05,),
                           "d40312df86619c7c8f24e7539d57eda67d3d7a7d6a66923cd0d58e98ef94f60f"),
    "C2 4096^2 25% N=512": ("workload_spmm_sweep", (0.25,),
                            "7abe14e2d4def1b0049227e9b92553711b6eb6db3c664c706a3c0012235967c7"),
    "C2 4096^2 50% N=512": ("workload_spmm_sweep", (0.5,),
                            "1c2e514e9764db301ace222cfb07c0fcd7d44aa792f234998a988c0ade361149"),
    "C3 SDDMM 4096^2 10% K=256": ("workload_sddmm", (),
                                  "ba2870f435580c302787e0a51a15068fe279c825bc3bd2be5a4fbf2951d00b44"),
    "C4 skewed 16384^2 Zipf(1.2) N=1024": ("workload_spmm_skewed", (),
                                           "84631048ba0ce5f73802ccf041ee5e5fdeb8b47b375b05f34cec155d964ef58d"),
    "C5 attention seq 8192 d 128": ("workload_attention", (),
                                    "0c9d5ee82a99fd50625bbfc2a74e40f485a0cb150cb0d8992185964e49f3cc41"),
    "8192^3 256x256 25%": ("workload_spmm_large_blocks", (0.25,),
                           "b01622720480ffb59720d13eaedeca59851d9dccc65f14772b4ec96dbf17c063"),
    "SpGEMM 8192^2 5% x 5%": ("workload_spgemm", (),
                              "83845a1f63727515fd1569dfcf4982376422925d944f26fca6a857af7d430a48"),
}


@pytest.mark.parametrize("name", sorted(DIGESTS))
def test_workload_digest(name):
    fn, args, digest = DIGESTS[name]
    assert W.workload_digest(getattr(W, fn)(*args)) == digest, name


def _xoshiro_reference(seed, lanes, lane, n):
    """Lane `lane` of workloads.Rng(seed, lanes) for n steps, in Python
    integers: splitmix64 from seed*lanes + lane, then xoshiro256**."""
    m = (1 << 64) - 1
    x = (seed * lanes + lane) & m
    s = []
    for _ in range(4):
        x = (x + 0x9E3779B97F4A7C15) & m
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        s.append(z ^ (z >> 31))
    rotl = lambda v, k: ((v << k) | (v >> (64 - k))) & m
    out = []
    for _ in range(n):
        out.append((rotl((s[1] * 5) & m, 7) * 9) & m)
        t = (s[1] << 17) & m
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
    return out


def test_xoshiro_streams_match_the_recurrence():
    r = W.Rng(12345, lanes=8)
    got = r.u64(8 * 20).reshape(20, 8)
    for lane in (0, 3, 7):
        assert [int(v) for v in got[:, lane]] == _xoshiro_reference(12345, 8, lane, 20)


def test_splitmix_seed_of_zero_gives_the_published_first_output():
    # splitmix64 seeded with 0: first output 0xE220A8397B1DCDAF (Vigna's
    # reference implementation, splitmix64.c); lane 0 of Rng(0) starts its
    # state with it.
    r = W.Rng(0, lanes=1)
    assert int(r.s[0][0]) == 0xE220A8397B1DCDAF


def test_sample_is_a_sorted_subset_and_uniform():
    r = W.Rng(7, lanes=1024)
    s = r.sample(100, 30)
    assert s.size == 30 and np.all(np.diff(s) > 0) and s.min() >= 0 and s.max() < 100
    counts = np.zeros(20, np.int64)
    for _ in range(2000):
        counts += np.bincount(r.sample(20, 5), minlength=20)
    # each position is picked with probability 1/4: 500 expected, sd ~19
    assert np.all(np.abs(counts - 500) < 100), counts


def test_uniform_and_normal_moments():
    r = W.Rng(9)
    u = r.random(200000, dtype=np.float32)
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.005 and abs(u.var() - 1 / 12) < 0.002
    z = r.standard_normal(200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
