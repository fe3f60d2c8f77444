"""Gather+attention half on the GPU through the C ABI: outputs against the oracle's exact fp64 attention on the same
fp16 operands (tolerance 2e-3 relative, max-abs), and the invariances the reference relies on or that this build
adds: T-invariance, split/grid invariance, page-permutation invariance, q8 rings on q8 sides change nothing."""
import numpy as np
import pytest

from kvcase import HD, NH, NKV, append_all, expected_attention, rel_err, synth_kv

pytestmark = pytest.mark.gpu
TOL = 2e-3


def run_attend(torch, st, Q, seqs, lens, T, layer0=0, nl=None):
    """Q [nl][nseq][T][24][256] numpy -> out numpy, same shape."""
    nl = nl or Q.shape[0]
    q = torch.from_numpy(np.ascontiguousarray(Q, np.float32)).cuda()
    out = torch.full_like(q, float("nan"))
    st.attend(layer0, nl, seqs, lens, T, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def layer_fmt(st, l):
    return st.kbits[l], st.vbits[l], st.krot[l], st.vrot[l]


def check_case(qkv, oracle, torch, spec, win, L, T, nl=1, seed=0, outliers=False, layers_checked=None):
    rng = np.random.default_rng(seed)
    K, V = synth_kv(rng, L, nl, outliers)
    st = qkv.KVStore(spec, win=win, n_layers=nl, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[4096] * 64)
    Q = rng.standard_normal((nl, 1, T, NH, HD)).astype(np.float32)
    out = run_attend(torch, st, Q, [0], [L], T)
    assert np.isfinite(out).all()
    ws = qkv.window_start(L, win)
    for l in (layers_checked if layers_checked is not None else range(nl)):
        kb, vb, kr, vr = layer_fmt(st, l)
        ref = expected_attention(oracle, Q[l, 0], K[:, l], V[:, l], T, kr, vr, kb, vb, ws, win > 0 and kb != 8,
                                 win > 0 and vb != 8)
        e = rel_err(out[l, 0], ref)
        assert e <= TOL, (spec, L, T, l, e)
    return st, out, (K, V, Q)


def test_cfg1_q8_4096(qkv, oracle, torch_gpu):
    """The reference host path's workload: all q8, one layer, 4,096 positions, one query token, seed 0."""
    check_case(qkv, oracle, torch_gpu, "", 0, 4096, 1, seed=0)


@pytest.mark.parametrize("spec", ["K*=5r,V*=6", "K*=5r,V*=5"])
def test_preset_f_window(qkv, oracle, torch_gpu, spec):
    """Preset F (K5r/V6 as benchmarked, and the reference's K5r/V5) with the 2,048 window: mixed ring/packed tiles."""
    check_case(qkv, oracle, torch_gpu, spec, 2048, 5000, 1, nl=2, seed=1, outliers=True)


@pytest.mark.parametrize("L", [1, 31, 33, 640, 1025, 2047])
def test_short_and_ragged(qkv, oracle, torch_gpu, L):
    check_case(qkv, oracle, torch_gpu, "K*=5r,V*=6", 512, L, 1, seed=L)


def test_verify_T8_q8(qkv, oracle, torch_gpu):
    """The verify shape (T = 8, causal among the 8, all q8), at a shorter context, seed 3."""
    check_case(qkv, oracle, torch_gpu, "", 0, 3000, 8, seed=3)


@pytest.mark.parametrize("T", [2, 3, 5, 8])
def test_verify_mixed(qkv, oracle, torch_gpu, T):
    L = 3190  # ws = 1280 (mixed ring / packed); rows L-T .. L-1 share one 640-bucket
    check_case(qkv, oracle, torch_gpu, "K*=5r,V*=6", 1024, L, T, seed=T, outliers=True)


def test_rotated_v_and_mixed_layers(qkv, oracle, torch_gpu):
    check_case(qkv, oracle, torch_gpu, "K0=4r,V0=7r,K1=8,V1=5,K2=6,V2=8r", 640, 2500, 2, nl=3, seed=5)


@pytest.mark.parametrize("T", [2, 3, 5, 8])
def test_t_invariance(qkv, oracle, torch_gpu, T):
    """Token t of a T-row call equals a 1-row call at context n+t+1 (bitwise; bench/dattn_bench.cu:1140-1160).
    T = 2 runs the 16-row kernel, T = 3 the 24-row one, T = 5 and 8 the 8-wave kernel (a full and a ragged half of 24
    rows; two full halves)."""
    torch = torch_gpu
    L = 3190
    st, out, (K, V, Q) = check_case(qkv, oracle, torch, "K*=5r,V*=6", 1024, L, T, seed=9 + T)
    for t in range(T):
        o1 = run_attend(torch, st, Q[:, :, t:t + 1], [0], [L - T + t + 1], 1)
        assert np.array_equal(o1[:, :, 0], out[:, :, t]), t


@pytest.mark.parametrize("spec,win,L,T", [("K*=5r,V*=6", 2048, 20000, 8), ("", 0, 9001, 5), ("K*=4,V*=7r", 640, 17001, 6),
                                          ("K0=8,V0=8,K1=6r,V1=5", 1024, 3190, 8)])
def test_wide_equals_batched(qkv, oracle, torch_gpu, spec, win, L, T):
    """T >= 5 (25..48 rows per kv head): the one-pass 8-wave kernel gives the bits of two 24-row batches, with
    several tiles per wave, window tiles, a partial last tile, two layers and a capped grid."""
    torch = torch_gpu
    print(f"wide {spec} L={L} T={T}", flush=True)
    st, out, (K, V, Q) = check_case(qkv, oracle, torch, spec, win, L, T, nl=2, seed=13 + T, outliers=True, layers_checked=[1])
    st.config("wide", 0)
    assert np.array_equal(run_attend(torch, st, Q, [0], [L], T), out)
    st.config("wide", 1)
    st.config("max_blocks", 37)
    assert np.array_equal(run_attend(torch, st, Q, [0], [L], T), out)
    st.config("wide", 0)  # the row batches on a capped grid (workgroups walk the batch-paired work items)
    assert np.array_equal(run_attend(torch, st, Q, [0], [L], T), out)
    st.config("max_blocks", 0)


@pytest.mark.parametrize("spec,win,L,T,tiles", [("K*=5r,V*=6", 2048, 20000, 1, 1), ("", 0, 9001, 8, 3), ("K*=4,V*=7r", 640, 5000, 2, 64),
                                                ("K*=5r,V*=6", 2048, 20000, 8, 2)])
def test_prefetch_changes_nothing(qkv, oracle, torch_gpu, spec, win, L, T, tiles):
    """mk_kv_prefetch (the attention's first tiles read into L2, on another stream) leaves every output bit as it was,
    with window tiles, more tiles than a slice holds, two layers, and T = 8 as two 24-row batches (work items of the
    attention launch that name the same segments); bad tile counts are refused."""
    torch = torch_gpu
    print(f"prefetch {spec} L={L} T={T} tiles={tiles}", flush=True)
    st, out, (K, V, Q) = check_case(qkv, oracle, torch, spec, win, L, T, nl=2, seed=31 + T, layers_checked=[])
    side = torch.cuda.Stream()
    st.prefetch(0, 2, [0], [L], T, tiles, side.cuda_stream)
    side.synchronize()
    assert np.array_equal(run_attend(torch, st, Q, [0], [L], T), out)
    for bad in (0, 65):
        with pytest.raises(qkv.KVError, match="tiles"):
            st.prefetch(0, 2, [0], [L], T, bad)
    with pytest.raises(qkv.KVError, match="context length"):
        st.prefetch(0, 2, [0], [L + 1], T)


def test_grid_invariance(qkv, oracle, torch_gpu):
    """Outputs do not depend on the launch geometry (max_blocks = split count of the grid), bitwise."""
    torch = torch_gpu
    st, out, (K, V, Q) = check_case(qkv, oracle, torch, "K*=5r,V*=6", 2048, 7000, 1, nl=2, seed=6)
    for mb in (1, 3, 17, 64, 1000):
        st.config("max_blocks", mb)
        assert np.array_equal(run_attend(torch, st, Q, [0], [7000], 1), out), mb
    st.config("max_blocks", 0)
    assert np.array_equal(run_attend(torch, st, Q, [0], [7000], 1), out)


@pytest.mark.parametrize("spec,win,L", [("K*=5r,V*=6", 2048, 7001), ("K*=4,V*=7r", 640, 5000), ("K*=4r,V*=4", 256, 3333),
                                        ("K*=6,V*=5r", 2048, 4100)])
def test_occupancy_invariance(qkv, oracle, torch_gpu, spec, win, L):
    """Three workgroups per CU (stages of one packed tile; q8 window tiles copied in two halves) give the same bits as
    two, with window tiles, a partial last tile and two layers in the launch; occupancy 0 picks by launch size."""
    torch = torch_gpu
    st, out, (K, V, Q) = check_case(qkv, oracle, torch, spec, win, L, 1, nl=2, seed=11, outliers=True)
    for occ in (3, 2, 0, 3):
        st.config("occupancy", occ)
        assert np.array_equal(run_attend(torch, st, Q, [0], [L], 1), out), occ
    st.config("occupancy", 0)


def test_ring_on_q8_sides_changes_nothing(qkv, oracle, torch_gpu):
    """MK_KV_WIN_ALL (loader.cu:1487-1490): q8 rings on q8 sides give byte-identical outputs."""
    torch = torch_gpu
    rng = np.random.default_rng(7)
    L = 5000
    K, V = synth_kv(rng, L, 1)
    Q = rng.standard_normal((1, 1, 1, NH, HD)).astype(np.float32)
    a = qkv.KVStore("", win=1024, win_all=1, n_layers=1, ctx=L)
    b = qkv.KVStore("", win=0, n_layers=1, ctx=L)
    append_all(torch, a, 0, K, V)
    append_all(torch, b, 0, K, V)
    assert np.array_equal(run_attend(torch, a, Q, [0], [L], 1), run_attend(torch, b, Q, [0], [L], 1))


def test_multi_sequence_paged(qkv, oracle, torch_gpu):
    """Config 5's shape at reduced lengths: several sequences, 256-position pages under a random permutation; each
    sequence matches the oracle and equals the same data in a contiguous store bit for bit."""
    torch = torch_gpu
    rng = np.random.default_rng(8)
    lens = [700, 2300, 3100]
    ctx, page = 3328, 256
    npg = ctx // page
    st = qkv.KVStore("K*=5r,V*=6", win=1024, n_layers=2, n_seq=3, ctx=ctx, page=page, n_pages=3 * npg)
    perm = rng.permutation(3 * npg)
    data = []
    for s, L in enumerate(lens):
        st.set_pages(s, perm[s * npg:(s + 1) * npg])
        K, V = synth_kv(rng, L, 2, outliers=True)
        append_all(torch, st, s, K, V, chunks=[1000, 1, 1000, 5000])
        data.append((K, V))
    Q = rng.standard_normal((2, 3, 1, NH, HD)).astype(np.float32)
    out = run_attend(torch, st, Q, [0, 1, 2], lens, 1)
    for s, L in enumerate(lens):
        K, V = data[s]
        ws = qkv.window_start(L, 1024)
        for l in range(2):
            ref = expected_attention(oracle, Q[l, s], K[:, l], V[:, l], 1, 1, 0, 5, 6, ws, True, True)
            assert rel_err(out[l, s], ref) <= TOL, (s, l)
        flat = qkv.KVStore("K*=5r,V*=6", win=1024, n_layers=2, ctx=ctx)
        append_all(torch, flat, 0, K, V)
        assert np.array_equal(run_attend(torch, flat, Q[:, s:s + 1], [0], [L], 1)[:, 0], out[:, s]), s


@pytest.mark.parametrize("T", [1, 8])
def test_prefetch_multi_sequence_paged(qkv, oracle, torch_gpu, T):
    """mk_kv_prefetch over several paged sequences (work items of three sequences, page-table lookups) changes no output
    bit, at T = 1 and at T = 8 (row batches)."""
    torch = torch_gpu
    rng = np.random.default_rng(80 + T)
    lens = [900, 2300, 3100]
    ctx, page = 3328, 256
    npg = ctx // page
    st = qkv.KVStore("K*=5r,V*=6", win=1024, n_layers=2, n_seq=3, ctx=ctx, page=page, n_pages=3 * npg)
    perm = rng.permutation(3 * npg)
    for s, L in enumerate(lens):
        st.set_pages(s, perm[s * npg:(s + 1) * npg])
        K, V = synth_kv(rng, L, 2, outliers=True)
        append_all(torch, st, s, K, V, chunks=[2048] * 2)
    Q = rng.standard_normal((2, 3, T, NH, HD)).astype(np.float32)
    out = run_attend(torch, st, Q, [0, 1, 2], lens, T)
    assert np.isfinite(out).all()
    side = torch.cuda.Stream()
    st.prefetch(0, 2, [0, 1, 2], lens, T, 4, side.cuda_stream)
    side.synchronize()
    assert np.array_equal(run_attend(torch, st, Q, [0, 1, 2], lens, T), out)


def test_verify_multi_sequence_paged(qkv, oracle, torch_gpu):
    """T = 8 over three paged sequences of different lengths (the persistent verify kernel walks work items of several
    sequences and layers): bitwise equal to the two-batch kernel, also with a grid of 5 workgroups, and sequences 0 and
    2 within tolerance of the oracle."""
    torch = torch_gpu
    rng = np.random.default_rng(18)
    lens, T = [704, 17000, 20100], 8
    ctx, page = 20224, 256
    npg = ctx // page
    print(f"verify paged lens={lens}", flush=True)
    st = qkv.KVStore("K*=5r,V*=6", win=2048, n_layers=2, n_seq=3, ctx=ctx, page=page, n_pages=3 * npg)
    perm = rng.permutation(3 * npg)
    data = []
    for s, L in enumerate(lens):
        st.set_pages(s, perm[s * npg:(s + 1) * npg])
        K, V = synth_kv(rng, L, 2, outliers=True)
        append_all(torch, st, s, K, V, chunks=[4096] * 8)
        data.append((K, V))
    Q = rng.standard_normal((2, 3, T, NH, HD)).astype(np.float32)
    out = run_attend(torch, st, Q, [0, 1, 2], lens, T)
    for s in (0, 2):
        K, V = data[s]
        ref = expected_attention(oracle, Q[1, s], K[:, 1], V[:, 1], T, 1, 0, 5, 6, qkv.window_start(lens[s], 2048), True, True)
        assert rel_err(out[1, s], ref) <= TOL, s
    st.config("wide", 0)
    assert np.array_equal(run_attend(torch, st, Q, [0, 1, 2], lens, T), out)
    st.config("wide", 1)
    st.config("max_blocks", 5)
    assert np.array_equal(run_attend(torch, st, Q, [0, 1, 2], lens, T), out)
    st.config("max_blocks", 0)


def test_attend_errors(qkv, torch_gpu):
    st = qkv.KVStore("K*=5r,V*=6", win=1024, n_layers=1, ctx=4000)
    assert qkv.window_start(3201, 1024) != qkv.window_start(3194, 1024)
    with pytest.raises(qkv.KVError, match="straddle"):
        st.attend(0, 1, [0], [3201], 8, 1, 1)
    with pytest.raises(qkv.KVError, match="T must"):
        st.attend(0, 1, [0], [100], 9, 1, 1)
    with pytest.raises(qkv.KVError, match="context"):
        st.attend(0, 1, [0], [4001], 1, 1, 1)
    with pytest.raises(qkv.KVError, match="occupancy"):
        st.config("occupancy", 1)
    with pytest.raises(qkv.KVError, match="wide"):
        st.config("wide", 3)
    with pytest.raises(qkv.KVError, match="wide"):
        st.config("wide", -1)
    with pytest.raises(qkv.KVError, match="unknown knob"):
        st.config("no_such_knob", 0)


def test_attend_rejects_unstored_and_evicted_rows(qkv, torch_gpu):
    """A context past the stored rows, or one whose window rows later appends have overwritten in the ring, is
    refused through the C ABI (mk_last_error); after a rewind to that length the call runs."""
    torch = torch_gpu
    rng = np.random.default_rng(17)
    K, V = synth_kv(rng, 5000, 1)
    st = qkv.KVStore("K*=5r,V*=6", win=640, n_layers=1, ctx=6000)
    append_all(torch, st, 0, K, V)
    q = torch.zeros(1, 1, 1, NH, HD, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(qkv.KVError, match="beyond the 5000 positions stored"):
        st.attend(0, 1, [0], [5001], 1, q.data_ptr(), out.data_ptr())
    with pytest.raises(qkv.KVError, match="overwritten"):
        st.attend(0, 1, [0], [1000], 1, q.data_ptr(), out.data_ptr())
    st.attend(0, 1, [0], [5000], 1, q.data_ptr(), out.data_ptr())
    st.rewind(0, 1000)
    st.attend(0, 1, [0], [1000], 1, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    # a store without rings keeps every row: any stored length may be attended
    flat = qkv.KVStore("", n_layers=1, ctx=6000)
    append_all(torch, flat, 0, K, V)
    flat.attend(0, 1, [0], [1000], 1, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1, 8])
def test_eight_sequences_per_call(qkv, oracle, torch_gpu, T):
    """The most sequences one call takes (8) over a shared page pool, every sequence against the oracle; a ninth is
    refused."""
    torch = torch_gpu
    rng = np.random.default_rng(60 + T)
    lens = [int(x) for x in rng.integers(T + 40, 2400, 8)]
    lens = [L - (L % 640) + 600 if qkv.cap_T(L - T, T) < T else L for L in lens]  # the T rows inside one bucket
    ctx, page = 2560, 256
    npg = ctx // page
    st = qkv.KVStore("K*=5r,V*=6", win=512, n_layers=1, n_seq=9, ctx=ctx, page=page, n_pages=9 * npg)
    perm = rng.permutation(9 * npg)
    data = []
    for s in range(9):
        st.set_pages(s, perm[s * npg:(s + 1) * npg])
    for s, L in enumerate(lens):
        K, V = synth_kv(rng, L, 1, outliers=True)
        append_all(torch, st, s, K, V)
        data.append((K, V))
    Q = rng.standard_normal((1, 8, T, NH, HD)).astype(np.float32)
    out = run_attend(torch, st, Q, list(range(8)), lens, T)
    for s, L in enumerate(lens):
        K, V = data[s]
        ref = expected_attention(oracle, Q[0, s], K[:, 0], V[:, 0], T, 1, 0, 5, 6, qkv.window_start(L, 512), True, True)
        assert rel_err(out[0, s], ref) <= TOL, (s, L)
    K, V = synth_kv(rng, 100, 1)
    append_all(torch, st, 8, K, V)
    q9 = torch.zeros((1, 9, 1, NH, HD), device="cuda")
    with pytest.raises(qkv.KVError, match="sequences"):
        st.attend(0, 1, list(range(9)), lens + [100], 1, q9.data_ptr(), q9.data_ptr())


def test_layer_window_of_a_17_slot_store(qkv, oracle, torch_gpu):
    """A launch over slots 14..16 of a 17-slot store (the launch's first slot is not slot 0) equals the three one-slot
    calls bitwise, and slot 16 matches the oracle."""
    torch = torch_gpu
    rng = np.random.default_rng(71)
    L, nl = 3000, 17
    st = qkv.KVStore("K*=5r,V*=6", win=1024, n_layers=nl, ctx=L)
    K, V = synth_kv(rng, L, nl, outliers=True)
    append_all(torch, st, 0, K, V)
    Q = rng.standard_normal((3, 1, 1, NH, HD)).astype(np.float32)
    out = run_attend(torch, st, Q, [0], [L], 1, layer0=14, nl=3)
    for l in range(3):
        one = run_attend(torch, st, Q[l:l + 1], [0], [L], 1, layer0=14 + l, nl=1)
        assert np.array_equal(one[0], out[l]), l
    ref = expected_attention(oracle, Q[2, 0], K[:, 16], V[:, 16], 1, 1, 0, 5, 6, qkv.window_start(L, 1024), True, True)
    assert rel_err(out[2, 0], ref) <= TOL
