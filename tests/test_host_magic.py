"""The division-free index arithmetic of the decode kernels (kv_launch.h magic31, kv_attn_decode.h div_m):
floor(n / d) = (2 n * ceil(2^31 / d)) >> 32, checked exhaustively over the domains the kernels use it on -- work item
n < 65,536 (8 sequences x 16 layers x 4 kv heads x 128 segments) by segment count d = 1..128, query row n < 64 by
T = 1..8 -- and on random pairs with n d < 2^31, the bound the kernels' header states."""
import numpy as np


def magic31(d):
    return ((1 << 31) + d - 1) // d  # the host's formula, in exact integers


def div_m(n, M):
    return (2 * n.astype(np.uint64) * np.uint64(M)) >> np.uint64(32)


def test_segment_and_row_domains_exhaustive():
    n = np.arange(65536, dtype=np.uint64)
    for d in range(1, 129):
        assert magic31(d) < 2 ** 32
        assert np.array_equal(div_m(n, magic31(d)), n // np.uint64(d)), d
    r = np.arange(64, dtype=np.uint64)
    for T in range(1, 9):
        assert np.array_equal(div_m(r, magic31(T)), r // np.uint64(T)), T


def test_random_pairs_within_the_bound():
    rng = np.random.default_rng(0)
    d = rng.integers(1, 1 << 16, 200000, dtype=np.uint64)
    n = (rng.random(200000) * ((1 << 31) / d.astype(np.float64))).astype(np.uint64)
    n = np.minimum(n, ((1 << 31) - 1) // d)  # n d < 2^31
    M = np.array([magic31(int(x)) for x in d], dtype=np.uint64)
    got = (2 * n * M) >> np.uint64(32)
    assert np.array_equal(got, n // d)
