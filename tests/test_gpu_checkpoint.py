"""Park/unpark row copies and window-ring snapshots for exact checkpoint reuse (host_store.cu:80-160, ck_pool.cu's
MK_EXACT ring copies) through the C ABI: bit-for-bit round trips, and attention after a restore equal to attention
before the continuation."""
import numpy as np
import pytest

from kvcase import HD, NKV, NH, append_all, synth_kv

pytestmark = pytest.mark.gpu


def test_write_rows_round_trip(qkv, torch_gpu):
    rng = np.random.default_rng(21)
    nl, T = 2, 700
    K, V = synth_kv(rng, T, nl, outliers=True)
    a = qkv.KVStore("K*=5r,V*=6", win=256, n_layers=nl, ctx=1024)
    append_all(torch_gpu, a, 0, K, V, chunks=[300, 400])
    b = qkv.KVStore("K*=5r,V*=6", win=256, n_layers=nl, ctx=1024)
    for l in range(nl):
        for w in (0, 1):
            for g in range(NKV):
                q, s = a.read_rows(0, l, w, g, 0, T)
                b.write_rows(0, l, w, g, 0, q, s)
                q, s = a.read_rows(0, l, w, g, 0, T, ring=True)
                b.write_rows(0, l, w, g, 0, q, s, ring=True)
    assert a.digest(0) == b.digest(0)
    a.close()
    b.close()


def attend(torch, st, L, Q):
    q = torch.from_numpy(Q).cuda()
    out = torch.empty_like(q)
    st.attend(0, Q.shape[0], [0], [L], 1, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_ring_snapshot_restore_is_exact(qkv, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(22)
    nl, P, extra, win = 2, 1400, 800, 64
    K, V = synth_kv(rng, P + extra, nl, outliers=True)
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=nl, ctx=4096)
    append_all(torch, st, 0, K[:P], V[:P], chunks=[1000, 400])
    ws = qkv.window_start(P, win)
    assert 0 < ws < P
    before = {(l, w, g): st.read_rows(0, l, w, g, ws, P - ws, ring=True) for l in range(nl) for w in (0, 1) for g in range(NKV)}
    Q = rng.standard_normal((nl, 1, 1, NH, HD)).astype(np.float32)
    y0 = attend(torch, st, P, Q)
    snap = st.ring_snapshot(0)
    append_all(torch, st, 0, K[P:], V[P:], pos0=P)   # the continuation overwrites ring slots of the window
    changed = any(not np.array_equal(st.read_rows(0, l, w, g, ws, P - ws, ring=True)[0], before[(l, w, g)][0])
                  for l in range(nl) for w in (0, 1) for g in range(NKV))
    assert changed
    st.ring_restore(0, P, snap)
    for key, (q0, s0) in before.items():
        q, s = st.read_rows(0, key[0], key[1], key[2], ws, P - ws, ring=True)
        assert np.array_equal(q, q0) and np.array_equal(s, s0), key
    y1 = attend(torch, st, P, Q)
    assert np.array_equal(y0, y1)
    st.close()


def test_ring_restore_errors(qkv, torch_gpu):
    rng = np.random.default_rng(23)
    K, V = synth_kv(rng, 100, 1)
    a = qkv.KVStore("K*=5r,V*=6", win=64, n_layers=1, ctx=512)
    append_all(torch_gpu, a, 0, K, V)
    snap = a.ring_snapshot(0)
    with pytest.raises(qkv.KVError):
        a.ring_restore(0, 101, snap)          # beyond the snapshot's position
    b = qkv.KVStore("K*=5r,V*=6", win=64, n_layers=2, ctx=512)
    with pytest.raises(qkv.KVError):
        b.ring_restore(0, 50, snap)           # another store layout
    bad = snap.copy()
    bad[:8] = 0
    with pytest.raises(qkv.KVError):
        a.ring_restore(0, 50, bad)            # not a snapshot
    a.ring_restore(0, 50, snap)
    a.close()
    b.close()
