"""Prefill (mk_kv_prefill, mk_kv_prefill_prep) on the GPU: the chunk's causal attention over the mixed store within
2e-3 of the exact attention, bitwise independence from how the prompt is chunked, the stored rows bit-exact, decode
continuing after it, and the raw-projection form against the oracle's prep, gate and o_proj units."""
import numpy as np
import pytest

from kvcase import HD, NH, NKV, check_rows, expected_attention, rel_err, synth_kv

pytestmark = pytest.mark.gpu


def run_prefill(qkv, torch, spec, win, K, V, Q, chunks, ctx):
    """Prefill K/V [P][nl][4][256] with queries Q [nl][P][24][256] in the given chunks -> (store, out [nl][P][24][256])."""
    P, nl = K.shape[0], K.shape[1]
    st = qkv.KVStore(spec, win=win, n_layers=nl, ctx=ctx)
    outs, p = [], 0
    for c in chunks:
        k = torch.from_numpy(np.ascontiguousarray(K[p:p + c])).cuda()
        v = torch.from_numpy(np.ascontiguousarray(V[p:p + c])).cuda()
        q = torch.from_numpy(np.ascontiguousarray(Q[:, p:p + c])).cuda()
        o = torch.empty_like(q)
        print(f"prefill spec={spec!r} win={win} pos={p} T={c}", flush=True)
        st.prefill(0, 0, nl, p, c, k.data_ptr(), v.data_ptr(), 0, q.data_ptr(), o.data_ptr())
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
        p += c
    return st, np.concatenate(outs, axis=1)


def pieces(P):
    a, out = 0, []
    while a < P:
        b = min(P, (a // 640 + 1) * 640)
        out.append((a, b))
        a = b
    return out


@pytest.mark.parametrize("spec,win", [("K*=5r,V*=6", 512), ("", 0), ("K*=4,V*=5r", 1280)])
def test_prefill_parity_and_chunking(qkv, oracle, torch_gpu, spec, win):
    torch = torch_gpu
    rng = np.random.default_rng(41)
    P, nl = 2100, 2
    K, V = synth_kv(rng, P, nl, outliers=True)
    Q = rng.standard_normal((nl, P, NH, HD)).astype(np.float32)
    st, out = run_prefill(qkv, torch, spec, win, K, V, Q, [700, 1400], 4096)
    check_rows(oracle, st, K, V, ring_from=max(0, P - qkv.ring_rows(win)))
    for l in range(nl):
        kb, vb, kr, vr = st.kbits[l], st.vbits[l], st.krot[l], st.vrot[l]
        for a, b in pieces(P)[::2]:
            ws = qkv.window_start(b, win)
            ref = expected_attention(oracle, Q[l, a:b], K[:b, l], V[:b, l], b - a, kr, vr, kb, vb, ws, win > 0 and kb != 8,
                                     win > 0 and vb != 8)
            assert rel_err(out[l, a:b], ref) <= 2e-3, (l, a, b)
    st.close()
    for chunks in ([2100], [1, 639, 3, 1457]):
        st2, out2 = run_prefill(qkv, torch, spec, win, K, V, Q, chunks, 4096)
        assert np.array_equal(out2, out), chunks
        st2.close()


def test_prefill_two_segments_then_decode(qkv, oracle, torch_gpu):
    """A 9,000-position context (the last pieces over two key segments of 4,864 positions, the combine folding both),
    then a decode step on the same store."""
    torch = torch_gpu
    rng = np.random.default_rng(42)
    P, nl, win, spec = 9000, 1, 2048, "K*=5r,V*=6"
    K, V = synth_kv(rng, P + 1, nl, outliers=True)
    Q = rng.standard_normal((nl, P, NH, HD)).astype(np.float32)
    st, out = run_prefill(qkv, torch, spec, win, K[:P], V[:P], Q, [5000, 4000], 10240)
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    a, b = pieces(P)[-1]
    ref = expected_attention(oracle, Q[0, a:b], K[:b, 0], V[:b, 0], b - a, kr, vr, kb, vb, qkv.window_start(b, win), True, True)
    assert rel_err(out[0, a:b], ref) <= 2e-3
    st2, out2 = run_prefill(qkv, torch, spec, win, K[:P], V[:P], Q, [8200, 800], 10240)
    assert np.array_equal(out2, out)
    st2.close()
    # decode position P
    k = torch.from_numpy(np.ascontiguousarray(K[P:P + 1])).cuda()
    v = torch.from_numpy(np.ascontiguousarray(V[P:P + 1])).cuda()
    st.append(0, 0, 1, P, 1, k.data_ptr(), v.data_ptr(), 0)
    qd = rng.standard_normal((1, 1, 1, NH, HD)).astype(np.float32)
    q = torch.from_numpy(qd).cuda()
    o = torch.empty_like(q)
    st.attend(0, 1, [0], [P + 1], 1, q.data_ptr(), o.data_ptr())
    torch.cuda.synchronize()
    ref = expected_attention(oracle, qd[0, 0], K[:P + 1, 0], V[:P + 1, 0], 1, kr, vr, kb, vb, qkv.window_start(P + 1, win), True, True)
    assert rel_err(o.cpu().numpy()[0, 0], ref) <= 2e-3
    st.close()


def test_prefill_prep(qkv, oracle, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(43)
    P, nl, win, spec = 1000, 2, 512, "K*=5r,V*=5r"
    K, V = synth_kv(rng, P, nl)
    K *= 4.0
    QG = rng.standard_normal((nl, P, NH, 2 * HD)).astype(np.float32)
    KW = (1 + 0.2 * rng.standard_normal((nl, HD))).astype(np.float32)
    QW = (1 + 0.2 * rng.standard_normal((nl, HD))).astype(np.float32)
    table = oracle.rope_rows(0, P)
    Kp = np.empty_like(K)
    for t in range(P):
        for l in range(nl):
            for g in range(NKV):
                Kp[t, l, g] = oracle.qk_prep(K[t, l, g], KW[l], table[t])
    Qp = np.empty((nl, P, NH, HD), np.float32)
    for l in range(nl):
        for t in range(P):
            for h in range(NH):
                Qp[l, t, h] = oracle.qk_prep(QG[l, t, h, :HD], QW[l], table[t])
    st = qkv.KVStore(spec, win=win, n_layers=nl, ctx=1024)
    k, v, kw, qw, qg = (torch.from_numpy(a).cuda() for a in (K, V, KW, QW, QG))
    o = torch.empty((nl, P, NH, HD), device="cuda")
    xa = torch.zeros((nl, P, 192, 16), dtype=torch.int8, device="cuda")
    xb = torch.zeros_like(xa)
    m = torch.zeros((nl, P, 192, 4), dtype=torch.int16, device="cuda")
    st.prefill_prep(0, 0, nl, 0, P, k.data_ptr(), v.data_ptr(), kw.data_ptr(), qg.data_ptr(), qw.data_ptr(), o.data_ptr(), xa.data_ptr(),
                    xb.data_ptr(), m.data_ptr())
    torch.cuda.synchronize()
    check_rows(oracle, st, Kp, V, ring_from=max(0, P - qkv.ring_rows(win)))
    ref_st, y = run_prefill(qkv, torch, spec, win, Kp, V, Qp, [P], 1024)
    ref_st.close()
    o = o.cpu().numpy()
    og = oracle.gate(y, QG[..., HD:]).reshape(o.shape)
    assert np.abs(o - og).max() <= 1e-6 * np.abs(og).max()
    xa, xb, m = xa.cpu().numpy(), xb.cpu().numpy(), m.cpu().numpy().view(np.uint16)
    for l in range(nl):
        for t in range(0, P, 37):
            ea, eb, em = oracle.q32_row(o[l, t])
            assert np.array_equal(xa[l, t], ea) and np.array_equal(xb[l, t], eb) and np.array_equal(m[l, t], em), (l, t)
    st.close()


def test_prefill_errors(qkv, torch_gpu):
    torch = torch_gpu
    st = qkv.KVStore("", n_layers=1, ctx=256)
    x = torch.zeros((8, 1, NKV, HD), device="cuda")
    q = torch.zeros((1, 8, NH, HD), device="cuda")
    o = torch.empty_like(q)
    with pytest.raises(qkv.KVError):
        st.prefill(0, 0, 1, 16, 8, x.data_ptr(), x.data_ptr(), 0, q.data_ptr(), o.data_ptr())  # gap: nothing stored yet
    with pytest.raises(qkv.KVError):
        st.prefill(0, 0, 1, 250, 8, x.data_ptr(), x.data_ptr(), 0, q.data_ptr(), o.data_ptr())  # beyond ctx
    st.prefill(0, 0, 1, 0, 8, x.data_ptr(), x.data_ptr(), 0, q.data_ptr(), o.data_ptr())
    torch.cuda.synchronize()
    assert np.all(np.isfinite(o.cpu().numpy()))
    st.close()


@pytest.mark.parametrize("page", [256, 32, 96])
def test_prefill_paged_equals_contiguous(qkv, torch_gpu, page):
    """Prefill on a shared page pool with a permuted page table gives the contiguous store's outputs bit for bit.  The
    kernel's copy side follows its tiles from page to page: 32-position pages change page at every tile, and 96-position
    pages put the second key segment's start (position 1,024 of the last pieces) inside a page."""
    torch = torch_gpu
    rng = np.random.default_rng(44)
    P, nl, win, spec = 1500, 1, 512, "K*=5r,V*=6"
    K, V = synth_kv(rng, P, nl, outliers=True)
    Q = rng.standard_normal((nl, P, NH, HD)).astype(np.float32)
    st, ref = run_prefill(qkv, torch, spec, win, K, V, Q, [900, 600], 2048)
    st.close()
    npg = -(-2048 // page)
    paged = qkv.KVStore(spec, win=win, n_layers=nl, n_seq=2, ctx=2048, page=page, n_pages=2 * npg)
    perm = np.random.default_rng(7).permutation(2 * npg)
    paged.set_pages(1, perm[:npg])
    outs, p = [], 0
    for c in (900, 600):
        k = torch.from_numpy(np.ascontiguousarray(K[p:p + c])).cuda()
        v = torch.from_numpy(np.ascontiguousarray(V[p:p + c])).cuda()
        q = torch.from_numpy(np.ascontiguousarray(Q[:, p:p + c])).cuda()
        o = torch.empty_like(q)
        paged.prefill(1, 0, nl, p, c, k.data_ptr(), v.data_ptr(), 0, q.data_ptr(), o.data_ptr())
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
        p += c
    assert np.array_equal(np.concatenate(outs, axis=1), ref)
    paged.close()


@pytest.mark.parametrize("spec,win,win_all", [("K*=6r,V*=7", 640, 0), ("", 1024, 1)])
def test_prefill_after_appends(qkv, oracle, torch_gpu, spec, win, win_all):
    """Rows stored by decode-style appends, then a prefill chunk from that position (one-token piece included), then the
    exact attention of the chunk's rows; q8 sides with their own ring (win_all) as well."""
    torch = torch_gpu
    rng = np.random.default_rng(45)
    nl, P0, P = 1, 1279, 2000
    K, V = synth_kv(rng, P, nl, outliers=True)
    Q = rng.standard_normal((nl, P - P0, NH, HD)).astype(np.float32)
    st = qkv.KVStore(spec, win=win, n_layers=nl, ctx=2048, win_all=win_all)
    for p0, c in ((0, 1000), (1000, 279)):
        k = torch.from_numpy(np.ascontiguousarray(K[p0:p0 + c])).cuda()
        v = torch.from_numpy(np.ascontiguousarray(V[p0:p0 + c])).cuda()
        st.append(0, 0, nl, p0, c, k.data_ptr(), v.data_ptr(), 0)
    k = torch.from_numpy(np.ascontiguousarray(K[P0:])).cuda()
    v = torch.from_numpy(np.ascontiguousarray(V[P0:])).cuda()
    q = torch.from_numpy(Q).cuda()
    o = torch.empty_like(q)
    st.prefill(0, 0, nl, P0, P - P0, k.data_ptr(), v.data_ptr(), 0, q.data_ptr(), o.data_ptr())
    torch.cuda.synchronize()
    out = o.cpu().numpy()
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    ring_k = win > 0 and (kb != 8 or win_all)
    ring_v = win > 0 and (vb != 8 or win_all)
    for a, b in ((P0, 1280), (1280, 1920), (1920, P)):
        ref = expected_attention(oracle, Q[0, a - P0:b - P0], K[:b, 0], V[:b, 0], b - a, kr, vr, kb, vb, qkv.window_start(b, win),
                                 ring_k, ring_v)
        assert rel_err(out[0, a - P0:b - P0], ref) <= 2e-3, (a, b)
    st.close()
