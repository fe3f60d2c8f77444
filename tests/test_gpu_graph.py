"""A decode step's one-layer mk_kv_attend calls captured as a HIP graph and replayed (how a serving loop issues them):
every replay, with the program's own eager work and synchronizations between replays, gives the eager calls' output
bit for bit -- the attention and combine launches record no memset nodes.  Preset F (packed K5r/V6 with the q8
window) over several tiles per wave, T = 1 and T = 8 in both verify forms (two 24-row batches, the default, and the
persistent one-pass kernel)."""
import numpy as np
import pytest

from kvcase import HD, NH, append_all, synth_kv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,wide", [(1, 2), (8, 2), (8, 1)])
def test_graph_replay_equals_eager(qkv, torch_gpu, T, wide):
    torch = torch_gpu
    rng = np.random.default_rng(90 + T)
    L, nl = 20000, 3
    st = qkv.KVStore("K*=5r,V*=6", win=2048, n_layers=nl, ctx=L)
    st.config("wide", wide)
    K, V = synth_kv(rng, L, nl, outliers=True)
    append_all(torch, st, 0, K, V, chunks=[4096] * 8, f16=True)
    q = torch.from_numpy(rng.standard_normal((nl, 1, T, NH, HD)).astype(np.float32)).cuda()
    lay = q[0].numel() * 4
    eager = torch.full_like(q, float("nan"))
    for l in range(nl):
        st.attend(l, 1, [0], [L], T, q.data_ptr() + l * lay, eager.data_ptr() + l * lay)
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    assert np.isfinite(ref).all()
    out = torch.full_like(q, float("nan"))
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for l in range(nl):
                st.attend(l, 1, [0], [L], T, q.data_ptr() + l * lay, out.data_ptr() + l * lay, stream=side.cuda_stream)
    for rep in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"replay {rep}")
        # eager work between the replays (its partials share the store's workspace)
        st.attend(nl - 1, 1, [0], [L], T, q.data_ptr(), eager.data_ptr())
        torch.cuda.synchronize()


def test_graph_survives_workspace_growth(qkv, torch_gpu):
    """A graph captured over a small call keeps working after a larger eager call grows the store's workspace: the
    outgrown buffer stays allocated until the store is freed, so the replay's kernel arguments still point at live
    memory and the replay gives the eager bits."""
    torch = torch_gpu
    rng = np.random.default_rng(95)
    L, nl = 20000, 2
    st = qkv.KVStore("K*=5r,V*=6", win=2048, n_layers=nl, ctx=L)
    K, V = synth_kv(rng, L, nl, outliers=True)
    append_all(torch, st, 0, K, V, chunks=[4096] * 8, f16=True)
    q = torch.from_numpy(rng.standard_normal((1, 1, 1, NH, HD)).astype(np.float32)).cuda()
    eager = torch.full_like(q, float("nan"))
    st.attend(0, 1, [0], [L], 1, q.data_ptr(), eager.data_ptr())
    torch.cuda.synchronize()
    ref = eager.cpu().numpy()
    out = torch.full_like(q, float("nan"))
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st.attend(0, 1, [0], [L], 1, q.data_ptr(), out.data_ptr(), stream=side.cuda_stream)
    # both layers at T = 8: 16 times the partials of the captured call, so the workspace is reallocated
    big = torch.from_numpy(rng.standard_normal((nl, 1, 8, NH, HD)).astype(np.float32)).cuda()
    bout = torch.empty_like(big)
    st.attend(0, nl, [0], [L], 8, big.data_ptr(), bout.data_ptr())
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), ref, err_msg=f"replay {rep}")
