"""The oracle's Q/K prep (kvo_rope_rows, kvo_qk_prep) pinned by fp64 restatements of RMSNorm and rotate-half RoPE and
by closed forms."""
import numpy as np


def rope64(p, n):
    i = np.arange(32)
    th = (np.arange(p, p + n)[:, None].astype(np.float64)) * 1e7 ** (-2.0 * i / 64.0)
    return np.cos(th), np.sin(th)


def prep64(x, w, c, s):
    x = x.astype(np.float64)
    y = x / np.sqrt((x * x).mean() + 1e-6) * w.astype(np.float64)
    a, b = y[:32].copy(), y[32:64].copy()
    y[:32] = a * c - b * s            # rotate_half: x * cos + (-x2, x1) * sin over dims 0..63
    y[32:64] = b * c + a * s
    return y


def test_rope_table(oracle):
    t = oracle.rope_rows(0, 1)
    assert np.all(t[0, :, 0] == 1.0) and np.all(t[0, :, 1] == 0.0)
    for p0 in (1, 777, 131000):
        t = oracle.rope_rows(p0, 3)
        c, s = rope64(p0, 3)
        assert np.abs(t[..., 0] - c).max() <= 6e-8 and np.abs(t[..., 1] - s).max() <= 6e-8
        assert np.array_equal(t[..., 0], c.astype(np.float32))   # rounding the same double once


def test_prep_against_fp64(oracle):
    rng = np.random.default_rng(4)
    for p in (0, 3, 5000, 101599):
        x = (rng.standard_normal(256) * rng.uniform(0.1, 30)).astype(np.float32)
        w = (1 + 0.3 * rng.standard_normal(256)).astype(np.float32)
        rc = oracle.rope_rows(p, 1)[0]
        got = oracle.qk_prep(x, w, rc)
        ref = prep64(x, w, rc[:, 0].astype(np.float64), rc[:, 1].astype(np.float64))
        assert np.abs(got - ref).max() <= 2e-6 * np.abs(ref).max(), p
        # values 64.. are the RMSNorm alone; each rotated pair keeps its length
        n = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * w
        assert np.allclose(got[64:], n[64:], rtol=1e-6, atol=0)
        assert np.allclose(got[:32] ** 2 + got[32:64] ** 2, n[:32] ** 2 + n[32:64] ** 2, rtol=1e-5)


def test_prep_closed_forms(oracle):
    one = np.ones(256, np.float32)
    rc0 = oracle.rope_rows(0, 1)[0]
    got = oracle.qk_prep(np.full(256, 3.0, np.float32), one, rc0)      # constant row: c / sqrt(c^2 + eps)
    assert np.allclose(got, 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-7)
    x = np.zeros(256, np.float32)
    x[5] = 2.0                                                          # one value: 2 / sqrt(4 / 256 + eps), rotated
    rc = oracle.rope_rows(9, 1)[0]
    got = oracle.qk_prep(x, one, rc)
    a = 2.0 / np.sqrt(4.0 / 256 + 1e-6)
    assert np.isclose(got[5], a * rc[5, 0], rtol=1e-6) and np.isclose(got[37], a * rc[5, 1], rtol=1e-6)
    assert np.count_nonzero(got) == 2
