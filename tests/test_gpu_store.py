"""Append/evict half on the GPU through the C ABI: stored main rows, ring rows, scales, page-table gathers, rewind refill
and the state digest, bit for bit against the oracle."""
import numpy as np
import pytest

from kvcase import HD, NKV, append_all, check_rows, synth_kv

pytestmark = pytest.mark.gpu

SPECS = ["", "K*=5r,V*=6", "K*=5r,V*=5", "K*=4,V*=7r", "*=6r", "K0=8,V0=5r,K1=7,V1=4"]


@pytest.mark.parametrize("spec", SPECS)
@pytest.mark.parametrize("f16", [False, True])
def test_append_bit_exact(qkv, oracle, torch_gpu, spec, f16):
    torch = torch_gpu
    rng = np.random.default_rng(11)
    nl, T = 2, 300
    K, V = synth_kv(rng, T, nl, outliers=True)
    if f16:
        K, V = K.astype(np.float16).astype(np.float32), V.astype(np.float16).astype(np.float32)
    st = qkv.KVStore(spec, win=256, n_layers=nl, ctx=512)
    append_all(torch, st, 0, K, V, chunks=[1, 7, 64, 1000], f16=f16)
    check_rows(oracle, st, K, V)


def test_append_special_values(qkv, oracle, torch_gpu):
    """Zero blocks, |x| ties, huge and subnormal magnitudes."""
    torch = torch_gpu
    T = 8
    K = np.zeros((T, 1, NKV, HD), np.float32)
    V = np.zeros((T, 1, NKV, HD), np.float32)
    K[1, 0, 0, :32] = 2.0
    K[1, 0, 0, 5] = -2.0
    K[2, 0, 1, :] = 1e-41
    K[3, 0, 2, :] = np.linspace(-6e4, 6e4, HD)
    V[4, 0, 3, ::3] = -1.5
    V[5, 0, 0, :] = 3e38
    V[6, 0, 1, :] = np.tile([0.5, -0.5], 128)
    for spec in ("K*=5r,V*=6", "", "*=7"):
        st = qkv.KVStore(spec, win=64, n_layers=1, ctx=64)
        append_all(torch, st, 0, K, V)
        check_rows(oracle, st, K, V)


def test_ring_eviction(qkv, oracle, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(12)
    T = 3000
    K, V = synth_kv(rng, T, 1)
    st = qkv.KVStore("K*=5r,V*=6", win=512, n_layers=1, ctx=T)
    assert qkv.ring_rows(512) == 1312
    append_all(torch, st, 0, K, V, chunks=[8] * 40 + [5000])
    check_rows(oracle, st, K, V, ring_from=T - 1312)


def test_one_call_longer_than_the_ring(qkv, oracle, torch_gpu):
    """One append of about 3 ring lengths: positions p and p + kvrc of the same launch share a ring row, and only the
    newest kvrc positions may write it; the ring must hold exactly the last kvrc rows, whatever the dispatch order."""
    torch = torch_gpu
    rng = np.random.default_rng(16)
    kvrc = qkv.ring_rows(512)
    T = 3 * kvrc + 77
    K, V = synth_kv(rng, T, 2, outliers=True)
    st = qkv.KVStore("K*=5r,V0=6,V1=8", win=512, win_all=1, n_layers=2, ctx=T)
    append_all(torch, st, 0, K, V)
    check_rows(oracle, st, K, V, ring_from=T - kvrc)


def test_paged_gathers_and_digest(qkv, oracle, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(13)
    ctx, page = 1000, 64
    npg = -(-ctx // page)
    K0, V0 = synth_kv(rng, 900, 2)
    K1, V1 = synth_kv(rng, 700, 2)
    paged = qkv.KVStore("K*=5r,V*=6", win=256, n_layers=2, n_seq=2, ctx=ctx, page=page, n_pages=2 * npg + 3)
    perm = rng.permutation(2 * npg + 3)
    paged.set_pages(0, perm[:npg])
    paged.set_pages(1, perm[npg:2 * npg])
    append_all(torch, paged, 0, K0, V0, chunks=[100, 1, 63, 1000])
    append_all(torch, paged, 1, K1, V1, chunks=[256, 1000])
    check_rows(oracle, paged, K0, V0, seq=0)
    check_rows(oracle, paged, K1, V1, seq=1)
    flat = qkv.KVStore("K*=5r,V*=6", win=256, n_layers=2, n_seq=1, ctx=ctx)
    append_all(torch, flat, 0, K1, V1)
    assert paged.digest(1) == flat.digest(0)


def test_digest_layout(qkv, oracle, torch_gpu):
    """Header words and per-row hashes of the reference's layout (engine.cu:1436-1514), from oracle rows."""
    torch = torch_gpu
    rng = np.random.default_rng(14)
    T, nl = 1500, 2
    K, V = synth_kv(rng, T, nl)
    st = qkv.KVStore("K*=5r,V0=6", win=256, n_layers=nl, ctx=2048)
    append_all(torch, st, 0, K, V)
    kvrc = qkv.ring_rows(256)
    rlo = T - kvrc
    want = [0x4d4b444701, T, 0, kvrc, rlo, nl, NKV, 0]
    ring_words = []
    for l in range(nl):
        for w, X in ((0, K), (1, V)):
            bits = (st.vbits if w else st.kbits)[l]
            rot = (st.vrot if w else st.krot)[l]
            for g in range(NKV):
                mq, ms, rq, rs = oracle.store_rows(X[:, l, g], rot, bits, ring=True, threads=8)
                want += [oracle.row_digest(mq[p], bits, ms[p]) for p in range(T)]
                if bits != 8:
                    ring_words += [oracle.row_digest(rq[p], 8, rs[p]) for p in range(rlo, T)]
                else:
                    ring_words += [0] * (T - rlo)
    assert st.digest(0) == want + ring_words


def test_rewind_refills_ring(qkv, oracle, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(15)
    T = 2000
    K, V = synth_kv(rng, T, 1)
    st = qkv.KVStore("K*=5r,V*=6", win=512, n_layers=1, ctx=T)
    kvrc = qkv.ring_rows(512)
    append_all(torch, st, 0, K, V)
    P = 1500
    st.rewind(0, P)
    p0, p1 = max(0, P - kvrc), min(P, T - kvrc)
    assert p1 > p0
    for w, X, bits, rot in ((0, K, 5, 1), (1, V, 6, 0)):
        for g in range(NKV):
            mq, ms, _, _ = oracle.store_rows(X[:, 0, g], rot, bits, ring=False)
            q, s = st.read_rows(0, 0, w, g, p0, p1 - p0, ring=True)
            for i, p in enumerate(range(p0, p1)):
                rq, rs = oracle.ring_refill_row(mq[p], ms[p], bits)
                assert np.array_equal(q[i], rq) and np.array_equal(s[i], rs), (w, g, p)
            # rows p1 .. P-1 were not overwritten: still the appended q8 rows
            _, _, rq, rs = oracle.store_rows(X[:, 0, g], rot, bits, ring=True)
            q, s = st.read_rows(0, 0, w, g, p1, P - p1, ring=True)
            assert np.array_equal(q, rq[p1:P]) and np.array_equal(s, rs[p1:P])
    assert st.digest(0)[1] == P


def test_sizes(qkv, torch_gpu):
    st = qkv.KVStore("K*=5r,V*=6", win=2048, n_layers=16, ctx=4096)
    per_tok, rings, state, ck = st.sizes()
    assert per_tok == 16 * NKV * (160 + 16 + 192 + 16)
    assert rings == 16 * 2 * NKV * qkv.ring_rows(2048) * (HD + 16)
    assert state == 0 and ck == 0


def test_append_errors(qkv, torch_gpu):
    st = qkv.KVStore("", n_layers=2, ctx=100)
    with pytest.raises(qkv.KVError, match="positions"):
        st.append(0, 0, 1, 99, 2, 1, 1, 0)
    with pytest.raises(qkv.KVError, match="layers"):
        st.append(0, 1, 2, 0, 1, 1, 1, 0)
    with pytest.raises(qkv.KVError, match="sequence"):
        st.append(1, 0, 1, 0, 1, 1, 1, 0)
