"""Shared helpers of the GPU parity tests: seeded synthetic K/V/Q, the store through the C ABI, and the oracle's
expected rows and attention outputs for the same inputs."""
import numpy as np

HD, NKV, NH, GQA = 256, 4, 24, 6


def synth_kv(rng, T, nl, outliers=False):
    """K, V of shape [T][nl][4][256] fp32.  outliers: 4 channels per kv head scaled x12 (the outlier-channel distribution of the append and 101,600-context workloads)."""
    K = rng.standard_normal((T, nl, NKV, HD)).astype(np.float32)
    V = rng.standard_normal((T, nl, NKV, HD)).astype(np.float32)
    if outliers:
        for g in range(NKV):
            ch = np.random.default_rng(1000 + g).choice(HD, 4, replace=False)
            K[:, :, g, ch] *= 12.0
    return K, V


def to_dev(torch, x, f16):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.half() if f16 else t.float()).cuda().contiguous()


def append_all(torch, st, seq, K, V, pos0=0, chunks=None, f16=False, layer0=0):
    """Append K/V [T][nl][4][256] in chunks through mk_kv_append."""
    T = K.shape[0]
    nl = K.shape[1]
    chunks = chunks or [T]
    p = 0
    keep = []
    for c in chunks:
        if p >= T:
            break
        c = min(c, T - p)
        k = to_dev(torch, K[p:p + c], f16)
        v = to_dev(torch, V[p:p + c], f16)
        keep += [k, v]
        st.append(seq, layer0, nl, pos0 + p, c, k.data_ptr(), v.data_ptr(), 1 if f16 else 0)
        p += c
    torch.cuda.synchronize()
    return keep


def expected_rows(oracle, X, rot, bits, ring):
    """Oracle rows of one (layer, side, head): X [L][256] fp32 -> main q/s, ring q/s."""
    return oracle.store_rows(X, rot, bits, ring=ring, threads=8)


def expected_kv(oracle, X, rot, bits, ws, has_ring):
    """The fp16 operands the attention sees for positions 0..L-1 of one (layer, side, head): main rows below ws, q8
    ring rows from ws on (sides without a ring are q8 in the main store)."""
    mq, ms, rq, rs = oracle.store_rows(X, rot, bits, ring=True, threads=8)
    out = oracle.dequant_rows(mq, ms, bits, f16=True)
    if has_ring and ws < X.shape[0]:
        out[ws:] = oracle.dequant_rows(rq[ws:], rs[ws:], 8, f16=True)
    return out


def expected_attention(oracle, Q, Kl, Vl, T, krot, vrot, kbits, vbits, ws, kring, vring):
    """Q [T][24][256], Kl/Vl [L][4][256] of one layer/sequence -> out [T][24][256] (fp64 exact attention on the
    fp16 operands; V un-rotated by the FWHT when V is stored rotated).  The 4 kv heads run on host threads (the
    oracle's C calls release the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    out = np.zeros((T, NH, HD), np.float32)
    R = GQA * T

    def head(g):
        K = expected_kv(oracle, Kl[:, g], krot, kbits, ws, kring)
        V = expected_kv(oracle, Vl[:, g], vrot, vbits, ws, vring)
        q = np.zeros((R, HD), np.float32)
        for r in range(R):
            q[r] = oracle.q_prep(Q[r % T, GQA * g + r // T], krot)
        return oracle.attn_exact(q, K, V, T)

    with ThreadPoolExecutor(NKV) as ex:
        ys = list(ex.map(head, range(NKV)))
    for g, y in enumerate(ys):
        for r in range(R):
            v = y[r]
            if vrot:
                v = oracle.fwht(v)
            out[r % T, GQA * g + r // T] = v
    return out


def check_rows(oracle, st, K, V, seq=0, pos0=0, ring_from=0):
    T, nl = K.shape[0], K.shape[1]
    for l in range(nl):
        for w, X in ((0, K), (1, V)):
            bits = (st.vbits if w else st.kbits)[l]
            rot = (st.vrot if w else st.krot)[l]
            has_ring = st.win > 0 and bits != 8
            for g in range(NKV):
                mq, ms, rq, rs = oracle.store_rows(X[:, l, g], rot, bits, ring=True, threads=8)
                q, s = st.read_rows(seq, l, w, g, pos0, T)
                assert np.array_equal(q, mq), (l, w, g, "main values")
                assert np.array_equal(s, ms), (l, w, g, "main scales")
                if has_ring and ring_from < T:
                    q, s = st.read_rows(seq, l, w, g, pos0 + ring_from, T - ring_from, ring=True)
                    assert np.array_equal(q, rq[ring_from:]), (l, w, g, "ring values")
                    assert np.array_equal(s, rs[ring_from:]), (l, w, g, "ring scales")


def rel_err(got, ref):
    return float(np.abs(got.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))
