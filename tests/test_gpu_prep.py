"""The Q/K prep fused into the append and attention kernels (mk_kv_append_prep, mk_kv_attend_prep, mk_kv_set_rope):
stored K rows bit-exact against the oracle's quantizers of the oracle's prep, the attention of the raw q_proj output
bit-identical to mk_kv_attend_gated of the oracle-prepped queries, and within 2e-3 of the exact attention."""
import numpy as np
import pytest

from kvcase import HD, NH, NKV, check_rows, expected_attention, rel_err, synth_kv

pytestmark = pytest.mark.gpu


def prep_rows(oracle, X, W, table, pos0):
    """X [T][nl][n][256] raw rows -> prepped (row t rotated by table row pos0 + t, layer l normed by W[l])."""
    out = np.empty_like(X)
    for t in range(X.shape[0]):
        for l in range(X.shape[1]):
            for g in range(X.shape[2]):
                out[t, l, g] = oracle.qk_prep(X[t, l, g], W[l], table[pos0 + t])
    return out


def test_append_prep_bit_exact(qkv, oracle, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(21)
    nl, T, pos0 = 2, 200, 300
    K, V = synth_kv(rng, T, nl, outliers=True)
    K *= 7.0
    W = (1 + 0.2 * rng.standard_normal((nl, HD))).astype(np.float32)
    st = qkv.KVStore("K*=5r,V*=6", win=256, n_layers=nl, ctx=1024)
    k, v, w = (torch.from_numpy(a).cuda() for a in (K, V, W))
    st.append_prep(0, 0, nl, pos0, T, k.data_ptr(), v.data_ptr(), w.data_ptr())
    torch.cuda.synchronize()
    table = oracle.rope_rows(0, 1024)
    check_rows(oracle, st, prep_rows(oracle, K, W, table, pos0), V, pos0=pos0)
    st.close()


def test_custom_rope_table(qkv, oracle, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(22)
    T = 40
    K, V = synth_kv(rng, T, 1)
    W = np.ones((1, HD), np.float32)
    table = rng.uniform(-1, 1, (64, 32, 2)).astype(np.float32)   # any rows: the kernels only index them
    st = qkv.KVStore("*=6", n_layers=1, ctx=64)
    tab = torch.from_numpy(table).cuda()
    st.set_rope(tab.data_ptr(), 64)
    k, v, w = (torch.from_numpy(a).cuda() for a in (K, V, W))
    st.append_prep(0, 0, 1, 10, T, k.data_ptr(), v.data_ptr(), w.data_ptr())
    torch.cuda.synchronize()
    check_rows(oracle, st, prep_rows(oracle, K, W, table, 10), V, pos0=10)
    with pytest.raises(qkv.KVError):
        st.append_prep(0, 0, 1, 40, T, k.data_ptr(), v.data_ptr(), w.data_ptr())  # rows 40..79 beyond the 64-row table
    st.close()


@pytest.mark.parametrize("spec,T,n_seq", [("K*=5r,V*=6", 1, 1), ("K*=4,V*=5r", 3, 2), ("K*=5r,V*=6", 8, 2)])
def test_attend_prep(qkv, oracle, torch_gpu, spec, T, n_seq):
    torch = torch_gpu
    rng = np.random.default_rng(23)
    nl, win = 2, 512
    lens = [1900, 1333][:n_seq]
    st = qkv.KVStore(spec, win=win, n_layers=nl, n_seq=n_seq, ctx=2048)
    table = oracle.rope_rows(0, 2048)
    KW = (1 + 0.2 * rng.standard_normal((nl, HD))).astype(np.float32)
    QW = (1 + 0.2 * rng.standard_normal((nl, HD))).astype(np.float32)
    kw, qw = torch.from_numpy(KW).cuda(), torch.from_numpy(QW).cuda()
    KV = []
    for s, L in enumerate(lens):
        K, V = synth_kv(rng, L, nl, outliers=True)
        k, v = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
        st.append_prep(s, 0, nl, 0, L, k.data_ptr(), v.data_ptr(), kw.data_ptr())
        KV.append((prep_rows(oracle, K, KW, table, 0), V))
    QG = rng.standard_normal((nl, n_seq, T, NH, 2 * HD)).astype(np.float32)
    QG[..., :HD] *= 5.0
    Qp = np.empty((nl, n_seq, T, NH, HD), np.float32)
    for l in range(nl):
        for s, L in enumerate(lens):
            for t in range(T):
                for h in range(NH):
                    Qp[l, s, t, h] = oracle.qk_prep(QG[l, s, t, h, :HD], QW[l], table[L - T + t])
    G = np.ascontiguousarray(QG[..., HD:])
    qg, qp, gate = (torch.from_numpy(a).cuda() for a in (QG, Qp, G))
    outs = []
    for fused in (True, False):
        o = torch.empty((nl, n_seq, T, NH, HD), device="cuda")
        xa = torch.zeros((nl, n_seq, T, 192, 16), dtype=torch.int8, device="cuda")
        xb = torch.zeros_like(xa)
        m = torch.zeros((nl, n_seq, T, 192, 4), dtype=torch.int16, device="cuda")
        if fused:
            st.attend_prep(0, nl, list(range(n_seq)), lens, T, qg.data_ptr(), qw.data_ptr(), o.data_ptr(), xa.data_ptr(), xb.data_ptr(),
                           m.data_ptr())
        else:
            st.attend_gated(0, nl, list(range(n_seq)), lens, T, qp.data_ptr(), gate.data_ptr(), o.data_ptr(), xa.data_ptr(),
                            xb.data_ptr(), m.data_ptr())
        torch.cuda.synchronize()
        outs.append([a.cpu().numpy() for a in (o, xa, xb, m)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    o = outs[0][0]
    for l in range(nl):
        kb, vb, kr, vr = st.kbits[l], st.vbits[l], st.krot[l], st.vrot[l]
        for s, L in enumerate(lens):
            K, V = KV[s]
            ws = qkv.window_start(L, win)
            ref = expected_attention(oracle, Qp[l, s], K[:, l], V[:, l], T, kr, vr, kb, vb, ws, kb != 8, vb != 8)
            refg = oracle.gate(ref, G[l, s]).reshape(ref.shape)
            assert rel_err(o[l, s], refg) <= 2e-3, (l, s)
    st.close()


def test_prep_errors(qkv, torch_gpu):
    torch = torch_gpu
    st = qkv.KVStore("", n_layers=1, ctx=64)
    x = torch.zeros((8, 1, NKV, HD), device="cuda")
    with pytest.raises(qkv.KVError):
        st.append_prep(0, 0, 1, 0, 8, x.data_ptr(), x.data_ptr(), 0)
    st.append_prep(0, 0, 1, 0, 8, x.data_ptr(), x.data_ptr(), torch.ones(HD, device="cuda").data_ptr())
    qg = torch.zeros((1, 1, 1, NH, 2 * HD), device="cuda")
    o = torch.empty((1, 1, 1, NH, HD), device="cuda")
    with pytest.raises(qkv.KVError):
        st.attend_prep(0, 1, [0], [8], 1, qg.data_ptr(), 0, o.data_ptr())
    torch.cuda.synchronize()
    st.close()
