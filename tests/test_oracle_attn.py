"""Pins of the oracle's window geometry, digest hash and attention (closed forms and the documented spot values)."""
import numpy as np
import pytest

HD = 256
MASK64 = (1 << 64) - 1


def test_window_spot_values(oracle):
    # docs/CONFIGURATION.md:190-193: with W = 2048 the q8 window holds 2,561 .. 3,200 positions
    spans = {L - oracle.ws(L, 2048) for L in range(3201, 20000)}
    assert min(spans) == 2561 and max(spans) == 3200
    assert oracle.kvrc(2048) == 3232                     # loader.cu:1479-1486
    assert oracle.ws(101600, 2048) == 98560               # L = 101,600, W = 2,048: ring 3,040 / packed 98,560
    assert [oracle.ws(L, 2048) for L in (23000, 60000, 262144)] == [19840, 56960, 259200]
    assert {oracle.kvrc(w) for w in range(1921, 2561)} == {3232}
    assert oracle.ws(5000, 0) == 0 and oracle.kvrc(0) == 0
    for L in range(1, 3200):
        assert oracle.ws(L, 2048) == 0


def test_cap_T_brute_force(oracle):
    for n in list(range(0, 2000, 7)) + [639, 640, 1279, 1280]:
        for T in range(1, 9):
            c = oracle.cap_T(n, T)
            buckets = [-(-(n + t + 1) // 640) for t in range(c)]
            assert 1 <= c <= T and len(set(buckets)) == 1
            if c < T:
                assert -(-(n + c + 1) // 640) != buckets[0]


def py_dg_hash(b, h=0xcbf29ce484222325):
    b = bytes(b)
    i = 0
    while i + 8 <= len(b):
        w = int.from_bytes(b[i:i + 8], "little")
        h = ((h ^ w) * 0x100000001b3) & MASK64
        h ^= h >> 31
        i += 8
    for x in b[i:]:
        h = ((h ^ x) * 0x100000001b3) & MASK64
    return h


def test_dg_hash_known_words(oracle):
    assert oracle.dg_hash(np.zeros(0, np.uint8)) == 0xcbf29ce484222325
    # inputs under 8 bytes take only the byte loop, which is FNV-1a 64: the published FNV-1a test vectors (the FNV
    # reference test suite of Fowler, Noll and Vo) pin it independently of any restatement
    for text, want in [(b"a", 0xaf63dc4c8601ec8c), (b"b", 0xaf63df4c8601f1a5), (b"foo", 0xdcb27518fed9d577),
                       (b"foob", 0xdd120e790c2512af), (b"fooba", 0xcac165afa2fef40a), (b"foobar", 0x85944171f73967e8)]:
        assert oracle.dg_hash(np.frombuffer(text, np.uint8)) == want, text
    one = ((0xcbf29ce484222325 ^ 0x61) * 0x100000001b3) & MASK64
    assert oracle.dg_hash(np.frombuffer(b"a", np.uint8)) == one
    w = int.from_bytes(b"abcdefgh", "little")
    h = ((0xcbf29ce484222325 ^ w) * 0x100000001b3) & MASK64
    h ^= h >> 31
    assert oracle.dg_hash(np.frombuffer(b"abcdefgh", np.uint8)) == h
    rng = np.random.default_rng(0)
    for n in (0, 7, 8, 160, 272):
        b = rng.integers(0, 256, n, dtype=np.uint8)
        assert oracle.dg_hash(b) == py_dg_hash(b)


def test_attn_exact_closed_forms(oracle):
    rng = np.random.default_rng(1)
    L, T = 50, 3
    R = 6 * T
    V = rng.standard_normal((L, HD)).astype(np.float32)
    q = rng.standard_normal((R, HD)).astype(np.float32)
    out = oracle.attn_exact(q, np.zeros((L, HD), np.float32), V, T)   # equal scores: mean of the visible rows
    for r in range(R):
        t = r % T
        np.testing.assert_allclose(out[r], V[:L - T + t + 1].mean(0), rtol=1e-5, atol=1e-6)
    K = np.zeros((L, HD), np.float32)
    K[7] = 50 * q[0]                                                   # one dominant key
    out = oracle.attn_exact(q[:1], K, V, 1)
    np.testing.assert_allclose(out[0], V[7], rtol=1e-5, atol=1e-6)
    out = oracle.attn_exact(q[:6], K[:1], V[:1], 1)                    # L = 1
    assert np.allclose(out, V[0])


def numpy_attention(q, K, V, T):
    L = K.shape[0]
    out = np.zeros((q.shape[0], HD))
    for r in range(q.shape[0]):
        lim = L - T + r % T + 1
        s = K[:lim].astype(np.float64) @ q[r].astype(np.float64)
        p = np.exp(s - s.max())
        out[r] = p @ V[:lim].astype(np.float64) / p.sum()
    return out


@pytest.mark.parametrize("L,T", [(1, 1), (33, 1), (700, 1), (4096, 1), (1300, 8), (2049, 2)])
def test_attn_chunked_vs_exact(oracle, L, T):
    rng = np.random.default_rng(L + T)
    R = 6 * T
    q = np.stack([oracle.q_prep(x, 0) for x in rng.standard_normal((R, HD)).astype(np.float32)])
    K = rng.standard_normal((L, HD)).astype(np.float16).astype(np.float32)
    V = rng.standard_normal((L, HD)).astype(np.float16).astype(np.float32)
    ex = oracle.attn_exact(q, K, V, T)
    np.testing.assert_allclose(ex, numpy_attention(q, K, V, T), rtol=0, atol=1e-5 * np.abs(ex).max())
    ch = oracle.attn_chunked(q, K, V, T, threads=4)
    assert np.abs(ch - ex).max() <= 2e-3 * np.abs(ex).max()
    assert np.array_equal(ch, oracle.attn_chunked(q, K, V, T, threads=1))


def test_q_prep(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(HD).astype(np.float32)
    assert np.array_equal(oracle.q_prep(x, 0), (x * np.float32(0.0625)).astype(np.float16).astype(np.float32))
    assert np.array_equal(oracle.q_prep(x, 1), (oracle.fwht(x) * np.float32(0.0625)).astype(np.float16).astype(np.float32))
