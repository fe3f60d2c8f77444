"""The oracle's combine epilogue (kvo_gate, kvo_q32_row) pinned by closed forms and known answers."""
import numpy as np


def test_gate_closed_forms(oracle):
    y = np.array([1.0, -3.5, 1e-3, 7.25], np.float32)
    assert np.array_equal(oracle.gate(y, np.zeros(4, np.float32)), y / 2)           # sigmoid(0) = 1/2
    assert np.array_equal(oracle.gate(y, np.full(4, 100.0, np.float32)), y)         # 1 + exp(-100) == 1 in fp32
    assert np.all(np.abs(oracle.gate(y, np.full(4, -100.0, np.float32))) < 1e-40)


def test_q32_known_answers(oracle):
    o = np.zeros(6144, np.float32)
    o[5 * 32 + 20] = -2.0            # block j = 5 (head 0, k = 5): one value -> -127, odd block -> b, half 1
    b9 = 9 * 32                      # block j = 9 (head 1, k = 1): amax 127 -> d = 1, ties round half away from 0
    o[b9:b9 + 4] = [127.0, 2.5, -2.5, 0.5]
    xa, xb, m = oracle.q32_row(o)
    assert not xa[0:4].any() and not xa[6:].any()
    gi = 8 * 0 + 2 * (5 >> 1) + 1
    assert xb[gi, 4] == -127 and np.count_nonzero(xb[gi]) == 1
    assert m[gi, 1] == oracle.f2h(np.float32(2.0) / np.float32(127.0)) and np.int16(m[gi, 3]) == -127
    assert m[gi, 0] == 0 and m[gi, 2] == 0                       # the even block of the unit (j = 4) is all zero
    gi = 8 * 1 + 2 * (1 >> 1) + 0
    assert list(xb[gi, :4]) == [127, 3, -3, 1]
    assert np.int16(m[gi, 3]) == 128 and m[gi, 1] == oracle.f2h(np.float32(1.0))
    assert not xb[gi + 1].any()


def test_q32_sums_and_range(oracle):
    rng = np.random.default_rng(9)
    o = (rng.standard_normal(6144) * rng.uniform(0.01, 10, 6144)).astype(np.float32)
    xa, xb, m = oracle.q32_row(o)
    for j in range(192):
        part = j & 1
        gi0 = 8 * (j >> 3) + 2 * ((j >> 1) & 3)
        blk = o[32 * j:32 * j + 32]
        d = np.float32(np.abs(blk).max()) / np.float32(127.0)
        q = np.concatenate([(xb if part else xa)[gi0], (xb if part else xa)[gi0 + 1]]).astype(np.int32)
        assert np.abs(q).max() == 127
        assert np.all(np.abs(q - blk / d) <= 0.5 + 1e-3)
        assert np.int16(m[gi0, 2 + part]) == q[:16].sum() and np.int16(m[gi0 + 1, 2 + part]) == q[16:].sum()
