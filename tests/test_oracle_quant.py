"""Pins of the CPU oracle's conversions, quantizers, packing and FWHT: closed forms, hand-computed known answers and
independent numpy computations (not the oracle's own formulas), so that a dropped term, a wrong sign, a wrong nibble
or bit position, or a wrong rounding mode fails a test."""
import numpy as np
import pytest

HD = 256


def f16bits(x):
    with np.errstate(over="ignore"):
        return int(np.array([x], np.float32).astype(np.float16).view(np.uint16)[0])


def h16(b):
    return float(np.array([b], np.uint16).view(np.float16)[0])


def test_f2h_matches_numpy_rne(oracle):
    rng = np.random.default_rng(1)
    xs = list(rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000).astype(np.float32))
    xs += [0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e30, -1e30, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
           3 * 2.0 ** -26, 2.0 ** -25 * 1.0000001, 6.1035156e-05, 6.097555e-05, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]
    for e in range(-24, 16):  # exact halfway cases: ties go to even
        for m in (0, 1, 2, 3, 1022, 1023):
            xs.append((1 + (2 * m + 1) * 2.0 ** -11) * 2.0 ** e)
    for x in np.array(xs, np.float32):
        assert oracle.f2h(x) == f16bits(x), x
    for b in list(range(0, 0x7c00, 37)) + [0x8001, 0xfbff, 0x03ff]:
        assert oracle.h2f(b) == h16(b)


# ---------------------------------------------------------------------------------------------------------------- q8
def test_q8_known_answers(oracle):
    v = np.zeros(HD, np.float32)
    v[0:5] = [127.0, 2.5, 3.5, -2.5, -127.0]  # am = 127 -> id = 1: ties to even 2.5 -> 2, 3.5 -> 4, -2.5 -> -2
    v[64] = -3.0                              # block 2: a single value -> code -127
    v[96:100] = [0.5, -0.25, 0.125, 1.0]      # block 3: am = 1 -> id = 127: 63.5 -> 64, -31.75 -> -32, 15.875 -> 16
    q, s = oracle.store_q8(v)
    assert list(q[0:5]) == [127, 2, 4, -2, -127]
    assert s[0] == 0x3c00                      # half(127 / 127)
    assert not q[32:64].any() and s[1] == 0     # zero block: codes 0, scale +0
    assert q[64] == -127 and not q[65:96].any()
    assert s[2] == f16bits(np.float32(3.0) / np.float32(127.0))
    assert list(q[96:100]) == [64, -32, 16, 127]


def test_q8_properties(oracle):
    rng = np.random.default_rng(2)
    for trial in range(200):
        v = (rng.standard_normal(HD) * rng.uniform(0.01, 100)).astype(np.float32)
        q, s = oracle.store_q8(v)
        for b in range(8):
            blk = v[32 * b:32 * b + 32].astype(np.float64)
            am = np.abs(blk).max()
            assert s[b] == f16bits(np.float32(am) / np.float32(127.0))
            ideal = blk * 127.0 / am
            c = q[32 * b:32 * b + 32].astype(np.float64)
            assert np.all(np.abs(c - ideal) <= 0.5 + 1e-4)   # nearest code (fp32 product: tiny slack at ties)
            assert np.abs(c).max() == 127


# ---------------------------------------------------------------------------------------------------------------- b-bit
def manual_pack(n, bits):
    """Pack 256 biased codes n (0 .. 2^bits - 1) by the documented layout, independently of the oracle."""
    hb = bits - 4
    out = np.zeros(32 * bits, np.uint8)
    for i in range(HD):
        w, k = divmod(i, 8)
        nib = n[i] & 15
        if k < 4:
            out[4 * w + k] |= nib
        else:
            out[4 * w + k - 4] |= nib << 4
        if hb:
            hv = int(n[i]) >> 4
            bit = hb * k
            for t in range(hb):
                if (hv >> t) & 1:
                    out[128 + w * hb + (bit + t) // 8] |= 1 << ((bit + t) % 8)
    return out


@pytest.mark.parametrize("bits", [4, 5, 6, 7])
def test_qn_known_answers(oracle, bits):
    h = 1 << (bits - 1)
    v = np.zeros(HD, np.float32)
    # block 0: max value +h -> d = -1, id = -1, n = trunc(h + 0.5 - v)
    blk = np.array([h, -h, 0, 1, -1, 2.5, -2.5, h - 0.5] + [0] * 24, np.float32)
    v[0:32] = blk
    # block 1: the largest magnitude is negative -> d = +1 ... sv = -h: d = -h / -h = 1, id = 1, n = trunc(v + h + .5)
    v[32:36] = [-h, 3, -3, 0.49]
    # block 2: |x| tie between -2 and +2: the larger value (+2) is the signed max
    v[64:67] = [-2.0, 2.0, 1.0]
    # block 3: all zero -> d = -0 (scale 0x8000), id = 0, n = h
    q, s = oracle.store_qn(v, bits)
    n = oracle.codes(q, bits) + h
    expect0 = [min(2 * h - 1, int(np.trunc(h + 0.5 - x))) for x in blk]
    assert list(n[0:32]) == expect0
    assert s[0] == f16bits(-1.0)
    assert list(n[32:36]) == [0, h + 3, h - 3, h]  # trunc(-h+h+.5)=0, trunc(h+3.5)=h+3, trunc(h-2.5)=h-3, trunc(h+.99)=h
    assert s[1] == f16bits(1.0)
    d2 = np.float32(2.0) / np.float32(-h)
    assert s[2] == f16bits(d2)
    assert n[65] == 0 and n[64] == min(2 * h - 1, 2 * h)
    assert s[3] == 0x8000 and np.all(n[96:128] == h)
    assert np.array_equal(q, manual_pack(n, bits))


@pytest.mark.parametrize("bits", [4, 5, 6, 7])
def test_qn_properties_and_layout(oracle, bits):
    rng = np.random.default_rng(10 + bits)
    h = 1 << (bits - 1)
    for trial in range(100):
        v = (rng.standard_normal(HD) * rng.uniform(0.01, 50)).astype(np.float32)
        q, s = oracle.store_qn(v, bits)
        n = oracle.codes(q, bits) + h
        assert n.min() >= 0 and n.max() <= 2 * h - 1
        assert np.array_equal(q, manual_pack(n, bits))
        for b in range(8):
            blk = v[32 * b:32 * b + 32].astype(np.float64)
            i = np.lexsort((blk, np.abs(blk)))[-1]      # largest |x|, ties -> larger x
            d = np.float32(blk[i]) / np.float32(-h)
            assert s[b] == f16bits(d)
            ideal = blk / float(d) + h                   # real-valued index before rounding
            c = n[32 * b:32 * b + 32]
            ok = np.floor(ideal + 0.5)
            assert np.all((np.abs(c - np.minimum(ok, 2 * h - 1)) <= 1) & (np.abs(c - ideal) <= 1.0 + 1e-6))
            # dequantized values (fp16 scale) within half a step, plus the scale's own rounding, except the clamped
            # extreme (the value opposite the signed max may sit one step past the last code)
            d16 = float(h16(s[b]))
            deq = (c - h) * d16
            err = np.abs(deq - blk)
            bound = 0.5 * abs(float(d)) + h * abs(d16 - float(d)) + 1e-6 * abs(blk[i])
            assert np.all(err <= bound + (c == 2 * h - 1) * abs(float(d)))


def test_q4_is_qn_at_4_bits_by_independent_q4(oracle):
    """kv_store_q4 (qwen38_mk.cu:2029-2046): nibble = min(15, trunc(v / d + 8.5)) with d = sv / -8 (fp32 FMA)."""
    rng = np.random.default_rng(5)
    for _ in range(50):
        v = rng.standard_normal(HD).astype(np.float32)
        q, s = oracle.store_qn(v, 4)
        n = np.zeros(HD, np.int64)
        for b in range(8):
            blk = v[32 * b:32 * b + 32]
            i = np.lexsort((blk, np.abs(blk)))[-1]
            d = np.float32(blk[i]) / np.float32(-8.0)
            idv = np.float32(1.0) / d
            prod = blk.astype(np.float64) * np.float64(idv) + 8.5   # exact, then one rounding = fma
            n[32 * b:32 * b + 32] = np.minimum(15, np.trunc(prod.astype(np.float32)))
        assert np.array_equal(q, manual_pack(n, 4))


def test_dequant_roundings(oracle):
    rng = np.random.default_rng(3)
    v = rng.standard_normal(HD).astype(np.float32) * 3
    for bits in (4, 5, 6, 7, 8):
        q, s = oracle.store(v, bits)
        c = oracle.codes(q, bits)
        d = np.repeat([h16(x) for x in s], 32).astype(np.float32)
        f32 = oracle.dequant(q, s, bits)
        assert np.array_equal(f32, (d * c.astype(np.float32)))
        f16 = oracle.dequant(q, s, bits, f16=True)
        assert np.array_equal(f16, (d * c.astype(np.float32)).astype(np.float16).astype(np.float32))


# ---------------------------------------------------------------------------------------------------------------- FWHT
def sylvester(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def test_fwht_basis_vectors_exact(oracle):
    H = sylvester(HD)
    for i in [0, 1, 2, 7, 100, 128, 255]:
        e = np.zeros(HD, np.float32)
        e[i] = 1.0
        y = oracle.fwht(e)
        j = np.arange(HD)
        sign = np.array([(-1) ** bin(i & jj).count("1") for jj in j], np.float32)
        assert np.array_equal(y, sign / 16)
        assert np.array_equal(y, (H[:, i] / 16).astype(np.float32))


def test_fwht_matches_matrix_and_is_involution(oracle):
    H = sylvester(HD) / 16.0
    rng = np.random.default_rng(4)
    for _ in range(20):
        v = rng.standard_normal(HD).astype(np.float32)
        y = oracle.fwht(v)
        ref = H @ v.astype(np.float64)
        assert np.abs(y - ref).max() <= 8 * np.finfo(np.float32).eps * np.abs(v).sum() / 16
        assert np.abs(oracle.fwht(y) - v).max() <= 1e-5 * np.abs(v).max()
        # linearity (exact for power-of-two scaling)
        assert np.array_equal(oracle.fwht(2 * v), 2 * y)


def test_fwht_stage_order_bits(oracle):
    """Inputs whose butterfly sums round differently depending on the stage order: the ascending-bit order is pinned by
    an fp64 emulation of the same order with fp32 rounding at every step."""
    rng = np.random.default_rng(6)
    v = (rng.standard_normal(HD) * 10.0 ** rng.integers(-3, 4, HD)).astype(np.float32)
    x = v.copy()
    m = 1
    while m < HD:
        idx = np.arange(HD)
        lo = idx[(idx & m) == 0]
        a, b = x[lo].copy(), x[lo | m].copy()
        x[lo] = (a + b).astype(np.float32)
        x[lo | m] = (a - b).astype(np.float32)
        m <<= 1
    assert np.array_equal(oracle.fwht(v), (x * np.float32(0.0625)).astype(np.float32))


# ---------------------------------------------------------------------------------------------------------------- rows
def test_store_row_ring_is_q8_of_rotated(oracle):
    rng = np.random.default_rng(7)
    v = rng.standard_normal(HD).astype(np.float32)
    mq, ms, rq, rs = oracle.store_row(v, 1, 5)
    r = oracle.fwht(v)
    q5, s5 = oracle.store_qn(r, 5)
    q8, s8 = oracle.store_q8(r)
    assert np.array_equal(mq, q5) and np.array_equal(ms, s5)
    assert np.array_equal(rq, q8.view(np.uint8)) and np.array_equal(rs, s8)


def test_ring_refill_is_q8_of_fp32_dequant(oracle):
    rng = np.random.default_rng(8)
    v = rng.standard_normal(HD).astype(np.float32)
    mq, ms, _, _ = oracle.store_row(v, 0, 6, ring=False)
    rq, rs = oracle.ring_refill_row(mq, ms, 6)
    q8, s8 = oracle.store_q8(oracle.dequant(mq, ms, 6))
    assert np.array_equal(rq, q8.view(np.uint8)) and np.array_equal(rs, s8)
    # a q8 main row re-stored as q8 is the same row (the reference's MK_KV_WIN_ALL invariant)
    q, s = oracle.store_q8(v)
    rq8, rs8 = oracle.ring_refill_row(q.view(np.uint8), s, 8)
    assert np.array_equal(rq8, q.view(np.uint8)) and np.array_equal(rs8, s)
