"""The HIP path against the committed golden vectors (tests/golden/kv_golden.npz) through the C ABI, with no CPU
arithmetic at run time: stored bytes and scales bit-exact, attention within 2e-3 of the fixture's fp64 output."""
import os

import numpy as np
import pytest

from kvcase import HD, NKV, rel_err

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kv_golden.npz")
TOL = 2e-3


@pytest.fixture(scope="module")
def gold():
    with np.load(G, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("rot", ["n", "r"])
@pytest.mark.parametrize("bits", [4, 5, 6, 7, 8])
def test_rows_match_golden(qkv, torch_gpu, gold, bits, rot):
    torch = torch_gpu
    x = gold["rows_x"]                      # [64][256] fp16 -> 16 positions x 4 kv heads
    T = x.shape[0] // NKV
    k = torch.from_numpy(x.reshape(T, 1, NKV, HD).copy()).cuda()
    r = "r" if rot == "r" else ""
    st = qkv.KVStore(f"K0={bits}{r},V0={bits}{r}", win=64, win_all=1, n_layers=1, ctx=64)
    st.append(0, 0, 1, 0, T, k.data_ptr(), k.data_ptr(), 1)
    torch.cuda.synchronize()
    for w in (0, 1):
        for g in range(NKV):
            q, s = st.read_rows(0, 0, w, g, 0, T)
            assert np.array_equal(q, gold[f"rows_{bits}{rot}_q"][g::NKV]), (w, g, "main values")
            assert np.array_equal(s, gold[f"rows_{bits}{rot}_s"][g::NKV]), (w, g, "main scales")
            q, s = st.read_rows(0, 0, w, g, 0, T, ring=True)
            assert np.array_equal(q, gold[f"rows_{rot}_rq"][g::NKV]), (w, g, "ring values")
            assert np.array_equal(s, gold[f"rows_{rot}_rs"][g::NKV]), (w, g, "ring scales")
    st.close()


def test_attention_matches_golden(qkv, torch_gpu, gold):
    torch = torch_gpu
    K, V, Q = gold["attn_K"], gold["attn_V"], gold["attn_Q"]
    L, win = int(gold["attn_L"]), int(gold["attn_win"])
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=1, ctx=L)
    k = torch.from_numpy(K.reshape(L, 1, NKV, HD).copy()).cuda()
    v = torch.from_numpy(V.reshape(L, 1, NKV, HD).copy()).cuda()
    st.append(0, 0, 1, 0, L, k.data_ptr(), v.data_ptr(), 1)
    q = torch.from_numpy(Q.reshape(1, 1, 1, 24, HD).copy()).cuda()
    out = torch.empty_like(q)
    st.attend(0, 1, [0], [L], 1, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    e = rel_err(out.cpu().numpy()[0, 0], gold["attn_y"])
    assert e <= TOL, e
    st.close()
