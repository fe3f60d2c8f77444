"""mk_kv_attend_noalloc through the C ABI: the same bits as mk_kv_attend on two calls in a row (the second smaller,
on a different store), the size limit of its per-device workspace refused with a message.  The partials of the
allocation-free call live in the library's own device array, so the two entry points share kernels but not memory."""
import numpy as np
import pytest

from kvcase import HD, NH, append_all, synth_kv

pytestmark = pytest.mark.gpu


def both(torch, st, Q, seqs, lens, T):
    q = torch.from_numpy(np.ascontiguousarray(Q, np.float32)).cuda()
    a = torch.full_like(q, float("nan"))
    b = torch.full_like(q, float("nan"))
    st.attend(0, Q.shape[0], seqs, lens, T, q.data_ptr(), a.data_ptr())
    st.attend_noalloc(0, Q.shape[0], seqs, lens, T, q.data_ptr(), b.data_ptr())
    torch.cuda.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


def test_noalloc_equals_attend(qkv, torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(21)
    # first call: 2 layers, 2 paged sequences, T = 8 at 20,000 positions (several tiles per wave)
    K, V = synth_kv(rng, 20000, 2, outliers=True)
    st = qkv.KVStore("K*=5r,V*=6", win=2048, n_layers=2, n_seq=2, ctx=20000, page=256)
    append_all(torch, st, 0, K, V, chunks=[4096] * 5)
    append_all(torch, st, 1, K[:9000], V[:9000], chunks=[4096] * 3)
    Q = rng.standard_normal((2, 2, 8, NH, HD)).astype(np.float32)
    a, b = both(torch, st, Q, [0, 1], [20000, 9000], 8)
    assert np.isfinite(a).all() and np.array_equal(a, b)
    # second call, smaller: a new store, one layer, one token at 3,000 positions
    K2, V2 = synth_kv(rng, 3000, 1)
    st2 = qkv.KVStore("", n_layers=1, ctx=3000)
    append_all(torch, st2, 0, K2, V2)
    Q2 = rng.standard_normal((1, 1, 1, NH, HD)).astype(np.float32)
    a2, b2 = both(torch, st2, Q2, [0], [3000], 1)
    assert np.isfinite(a2).all() and np.array_equal(a2, b2)


def test_noalloc_rejects_oversize(qkv, torch_gpu):
    """4 layers at T = 8 of a 40,000-position context need 79 MiB, more than the 64 MiB workspace: a clear error, nothing launched."""
    torch = torch_gpu
    st = qkv.KVStore("", n_layers=4, ctx=40000)
    K, V = synth_kv(np.random.default_rng(22), 40000, 4)
    append_all(torch, st, 0, K, V, chunks=[8192] * 5)
    q = torch.zeros(4, 1, 8, NH, HD, device="cuda")
    out = torch.zeros_like(q)
    with pytest.raises(qkv.KVError, match="workspace"):
        st.attend_noalloc(0, 4, [0], [40000], 8, q.data_ptr(), out.data_ptr())
    st.attend(0, 4, [0], [40000], 8, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
