"""mk_kv_append_attend (the step's K/V rows stored inside the attention launch) against mk_kv_append followed by
mk_kv_attend, through the C ABI: the same output bits, the same stored rows (digests), and the store keeps working
afterwards.  Covers new rows in a wave's first tile, rows straddling a segment boundary (two workgroups store them),
48 query rows (T = 8, the 8-wave kernel), several layers with different formats, paged sequences, and fp16 / fp32 inputs."""
import numpy as np
import pytest

from kvcase import HD, NH, NKV, append_all, synth_kv, to_dev

pytestmark = pytest.mark.gpu


def step_inputs(rng, nseq, T, nl):
    K = rng.standard_normal((nseq, T, nl, NKV, HD)).astype(np.float32)
    V = rng.standard_normal((nseq, T, nl, NKV, HD)).astype(np.float32)
    K[..., :4] *= 12.0
    return K, V


@pytest.mark.parametrize("spec,win,lens,T,nl,f16,page,wide", [
    ("K*=5r,V*=6", 2048, [20000], 1, 1, True, 0, 2),     # several tiles per wave, the new row in the last ring tile
    ("K*=5r,V*=6", 2048, [40], 1, 2, False, 0, 2),       # a short context: the new row in a wave's first tile
    ("", 0, [1027], 8, 1, True, 0, 1),                   # T = 8 (8-wave kernel), rows 1019..1026 straddle segment 1024
    ("", 0, [1027], 8, 1, True, 0, 2),                   # the same in the default form (two 24-row batches)
    ("K*=5r,V*=6", 2048, [20000], 8, 1, True, 0, 2),     # T = 8 on packed sides: two 24-row batches both store the rows
    ("K*=5r,V*=6", 2048, [20000], 8, 1, True, 0, 1),     # the same in one 8-wave pass
    ("K0=4r,V0=7r,K1=8,V1=5", 640, [3190], 3, 2, False, 0, 2),
    ("K*=5r,V*=6", 1024, [2300, 700, 3100], 2, 1, True, 256, 2),
])
def test_append_attend_equals_two_calls(qkv, torch_gpu, spec, win, lens, T, nl, f16, page, wide):
    torch = torch_gpu
    rng = np.random.default_rng(70 + T + len(lens))
    nseq, ctx = len(lens), max(lens) + 64
    kw = dict(win=win, n_layers=nl, n_seq=nseq, ctx=ctx, page=page, n_pages=0)
    a, b = qkv.KVStore(spec, **kw), qkv.KVStore(spec, **kw)
    b.config("wide", wide)
    if page:
        perm = rng.permutation(nseq * (-(-ctx // page)))
        npg = -(-ctx // page)
        for s in range(nseq):
            a.set_pages(s, perm[s * npg:(s + 1) * npg])
            b.set_pages(s, perm[s * npg:(s + 1) * npg])
    for s, L in enumerate(lens):  # the context before the step
        K0, V0 = synth_kv(rng, L - T, nl, outliers=True)
        append_all(torch, a, s, K0, V0, chunks=[4096] * 8)
        append_all(torch, b, s, K0, V0, chunks=[4096] * 8)
    K, V = step_inputs(rng, nseq, T, nl)
    if f16:
        K, V = K.astype(np.float16).astype(np.float32), V.astype(np.float16).astype(np.float32)
    Q = rng.standard_normal((nl, nseq, T, NH, HD)).astype(np.float32)
    q = torch.from_numpy(Q).cuda()
    out_a, out_b = torch.full_like(q, float("nan")), torch.full_like(q, float("nan"))
    # a: one append call per sequence, then the attend
    keep = []
    for s, L in enumerate(lens):
        kd, vd = to_dev(torch, K[s], f16), to_dev(torch, V[s], f16)
        keep += [kd, vd]
        a.append(s, 0, nl, L - T, T, kd.data_ptr(), vd.data_ptr(), 1 if f16 else 0)
    a.attend(0, nl, list(range(nseq)), lens, T, q.data_ptr(), out_a.data_ptr())
    # b: the fused call
    kd, vd = to_dev(torch, K, f16), to_dev(torch, V, f16)
    b.append_attend(0, nl, list(range(nseq)), lens, T, kd.data_ptr(), vd.data_ptr(), 1 if f16 else 0, q.data_ptr(), out_b.data_ptr())
    torch.cuda.synchronize()
    oa, ob = out_a.cpu().numpy(), out_b.cpu().numpy()
    assert np.isfinite(oa).all() and np.array_equal(oa, ob)
    for s in range(nseq):
        assert a.digest(s) == b.digest(s), s
    # the store goes on: another fused step equals another pair of calls
    K2, V2 = step_inputs(rng, nseq, 1, nl)
    Q2 = torch.from_numpy(rng.standard_normal((nl, nseq, 1, NH, HD)).astype(np.float32)).cuda()
    lens2 = [L + 1 for L in lens]
    if all(qkv.cap_T(L, 1) == 1 for L in lens):
        o2a, o2b = torch.empty_like(Q2), torch.empty_like(Q2)
        for s, L in enumerate(lens):
            kd2, vd2 = to_dev(torch, K2[s], False), to_dev(torch, V2[s], False)
            keep += [kd2, vd2]
            a.append(s, 0, nl, L, 1, kd2.data_ptr(), vd2.data_ptr(), 0)
        a.attend(0, nl, list(range(nseq)), lens2, 1, Q2.data_ptr(), o2a.data_ptr())
        kd2, vd2 = to_dev(torch, K2, False), to_dev(torch, V2, False)
        b.append_attend(0, nl, list(range(nseq)), lens2, 1, kd2.data_ptr(), vd2.data_ptr(), 0, Q2.data_ptr(), o2b.data_ptr())
        torch.cuda.synchronize()
        assert np.array_equal(o2a.cpu().numpy(), o2b.cpu().numpy())


def test_append_attend_errors(qkv, torch_gpu):
    torch = torch_gpu
    st = qkv.KVStore("K*=5r,V*=6", win=640, n_layers=1, ctx=4000)
    K, V = synth_kv(np.random.default_rng(79), 1000, 1)
    append_all(torch, st, 0, K, V)
    k = torch.zeros(1, 1, 1, NKV, HD, device="cuda")
    q = torch.zeros(1, 1, 1, NH, HD, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(qkv.KVError, match="gap"):
        st.append_attend(0, 1, [0], [1002], 1, k.data_ptr(), k.data_ptr(), 0, q.data_ptr(), out.data_ptr())
    with pytest.raises(qkv.KVError, match="null K/V"):
        st.append_attend(0, 1, [0], [1001], 1, k.data_ptr(), 0, 0, q.data_ptr(), out.data_ptr())
    st.append_attend(0, 1, [0], [1001], 1, k.data_ptr(), k.data_ptr(), 0, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    assert st.digest(0)[1] == 1001
