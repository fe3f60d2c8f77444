"""The combine epilogue on the GPU (mk_kv_attend_gated): the output gate against the oracle, and the int8 o_proj units
bit-exact against the oracle's q32_store of the GPU's own gated output."""
import numpy as np
import pytest

from kvcase import HD, NH, append_all, expected_attention, rel_err, synth_kv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("spec,T", [("K*=5r,V*=6", 1), ("K*=5r,V*=5r", 3), ("K*=5r,V*=6", 8)])
def test_gated_output_and_q32(qkv, oracle, torch_gpu, spec, T):
    torch = torch_gpu
    rng = np.random.default_rng(31)
    L, win, nl = 2100, 512, 1
    K, V = synth_kv(rng, L, nl, outliers=True)
    st = qkv.KVStore(spec, win=win, n_layers=nl, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[1500, 600])
    Q = rng.standard_normal((nl, 1, T, NH, HD)).astype(np.float32)
    Gt = (rng.standard_normal((nl, 1, T, NH, HD)) * 2).astype(np.float32)
    q, gate = torch.from_numpy(Q).cuda(), torch.from_numpy(Gt).cuda()
    y = torch.empty_like(q)
    o = torch.empty_like(q)
    xa = torch.zeros((nl, 1, T, 192, 16), dtype=torch.int8, device="cuda")
    xb = torch.zeros_like(xa)
    meta = torch.zeros((nl, 1, T, 192, 4), dtype=torch.int16, device="cuda")
    st.attend(0, nl, [0], [L], T, q.data_ptr(), y.data_ptr())
    st.attend_gated(0, nl, [0], [L], T, q.data_ptr(), gate.data_ptr(), o.data_ptr(), xa.data_ptr(), xb.data_ptr(), meta.data_ptr())
    torch.cuda.synchronize()
    y, o = y.cpu().numpy(), o.cpu().numpy()
    # the gate applied to the same attention output (expf of two libraries: within a few ulp)
    og = oracle.gate(y, Gt).reshape(o.shape)
    assert np.abs(o - og).max() <= 1e-6 * max(np.abs(og).max(), 1.0)
    # and against the exact attention
    ws = qkv.window_start(L, win)
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    ref = expected_attention(oracle, Q[0, 0], K[:, 0], V[:, 0], T, kr, vr, kb, vb, ws, kb != 8, vb != 8)
    assert rel_err(o[0, 0], oracle.gate(ref, Gt[0, 0]).reshape(ref.shape)) <= 2e-3
    xa, xb, meta = xa.cpu().numpy(), xb.cpu().numpy(), meta.cpu().numpy().view(np.uint16)
    for t in range(T):
        ea, eb, em = oracle.q32_row(o[0, 0, t])
        assert np.array_equal(xa[0, 0, t], ea) and np.array_equal(xb[0, 0, t], eb) and np.array_equal(meta[0, 0, t], em), t
    st.close()


def test_gated_errors(qkv, torch_gpu):
    torch = torch_gpu
    st = qkv.KVStore("", n_layers=1, ctx=64)
    K = np.zeros((8, 1, 4, HD), np.float32)
    append_all(torch, st, 0, K, K)
    q = torch.zeros((1, 1, 1, NH, HD), device="cuda")
    o = torch.empty_like(q)
    xa = torch.zeros((1, 1, 1, 192, 16), dtype=torch.int8, device="cuda")
    with pytest.raises(qkv.KVError):
        st.attend_gated(0, 1, [0], [8], 1, q.data_ptr(), 0, o.data_ptr())                 # no gate
    with pytest.raises(qkv.KVError):
        st.attend_gated(0, 1, [0], [8], 1, q.data_ptr(), q.data_ptr(), o.data_ptr(), xa.data_ptr())  # a without b / meta
    st.close()
