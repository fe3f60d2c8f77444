"""The benchmark workloads at their full sizes on the GPU, against the oracle (one or two layers each, the same kernels
and launch shapes as the bench's calls), plus crafted long-context cases that drive the multi-tile loop of a wave.

Above 16,384 positions a wave of the decode kernel streams more than one 32-position tile of its segment (seg_len
grows with the context's 640-bucket), so these cases run what the short tests cannot: the O * alpha rescale of the
online softmax against a finite running maximum, the next-tile copy overlapping the math, and a wave whose tiles
switch from the packed store to the q8 ring.  Tolerance 2e-3 relative (max-abs) against fp64 attention on the same
fp16 operands; equalities are bitwise.

Workloads (the reference's kvattn_bench matrix, bench/kvattn_bench.cu:399-401, runs the same kind of sizes):
  101,600 positions, preset F (K5r/V6 and K5r/V5), window 2,048, K with outlier channels, T = 1 and 8;
  T = 8 verify at 38,000 positions, all q8, seed 3;
  4 paged sequences {23,000; 23,000; 60,000; 262,144}, 256-position pages under a seeded permutation, preset F;
  the append workload: 16 layers x 512 steps x 8 positions, window 2,048, every stored row against the oracle.
"""
import numpy as np
import pytest

from kvcase import GQA, HD, NH, NKV, append_all, expected_attention, rel_err, synth_kv

pytestmark = pytest.mark.gpu
TOL = 2e-3


def f16_kv(rng, L, nl, outliers):
    """K/V rounded to fp16 (the bench appends fp16; halves the host-to-device traffic)."""
    K, V = synth_kv(rng, L, nl, outliers)
    return K.astype(np.float16).astype(np.float32), V.astype(np.float16).astype(np.float32)


def attend(torch, st, Q, seqs, lens, T, layer0=0):
    q = torch.from_numpy(np.ascontiguousarray(Q, np.float32)).cuda()
    out = torch.full_like(q, float("nan"))
    st.attend(layer0, Q.shape[0], seqs, lens, T, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def expect(oracle, qkv, st, Q, K, V, L, T, l, win):
    kb, vb, kr, vr = st.kbits[l], st.vbits[l], st.krot[l], st.vrot[l]
    return expected_attention(oracle, Q, K[:L, l], V[:L, l], T, kr, vr, kb, vb, qkv.window_start(L, win),
                              win > 0 and kb != 8, win > 0 and vb != 8)


@pytest.mark.parametrize("T", [1, 8])
def test_cfg3_full_context(qkv, oracle, torch_gpu, T):
    """101,600 positions, K5r/V6 with the 2,048 window (98,560 packed + 3,040 ring positions), two layers: the fused
    two-layer launch and the one-layer launches against the oracle and bitwise equal; occupancy 2 vs 3 equal."""
    torch = torch_gpu
    L, nl, win = 101600, 2, 2048
    print(f"cfg3 L={L} T={T}", flush=True)
    rng = np.random.default_rng(30 + T)
    K, V = f16_kv(rng, L, nl, outliers=True)
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=nl, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[8192] * 13, f16=True)
    Q = rng.standard_normal((nl, 1, T, NH, HD)).astype(np.float32)
    fused = attend(torch, st, Q, [0], [L], T)
    for l in range(nl):
        e = rel_err(fused[l, 0], expect(oracle, qkv, st, Q[l, 0], K, V, L, T, l, win))
        assert e <= TOL, (l, e)
        one = attend(torch, st, Q[l:l + 1], [0], [L], T, layer0=l)
        assert np.array_equal(one[0], fused[l]), l
    if T == 1:
        for occ in (3, 2):
            st.config("occupancy", occ)
            assert np.array_equal(attend(torch, st, Q, [0], [L], T), fused), occ
            assert np.array_equal(attend(torch, st, Q[:1], [0], [L], T), fused[:1]), occ
        st.config("occupancy", 0)


def test_cfg3_full_context_k5_v5(qkv, oracle, torch_gpu):
    """The reference's own preset F (V 5-bit) at 101,600 positions."""
    torch = torch_gpu
    L, win = 101600, 2048
    print(f"cfg3 K5r/V5 L={L}", flush=True)
    rng = np.random.default_rng(35)
    K, V = f16_kv(rng, L, 1, outliers=True)
    st = qkv.KVStore("K*=5r,V*=5", win=win, n_layers=1, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[8192] * 13, f16=True)
    Q = rng.standard_normal((1, 1, 1, NH, HD)).astype(np.float32)
    out = attend(torch, st, Q, [0], [L], 1)
    e = rel_err(out[0, 0], expect(oracle, qkv, st, Q[0, 0], K, V, L, 1, 0, win))
    assert e <= TOL, e


def test_cfg4_verify_38000(qkv, oracle, torch_gpu):
    """T = 8 verify (48 query rows per kv head, causal among the 8) at 38,000 positions, all q8, seed 3; token t
    equals a one-token call at its own length, bitwise."""
    torch = torch_gpu
    L, T = 38000, 8
    print(f"cfg4 L={L} T={T}", flush=True)
    rng = np.random.default_rng(3)
    K, V = f16_kv(rng, L, 1, outliers=False)
    st = qkv.KVStore("", n_layers=1, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[8192] * 5, f16=True)
    Q = rng.standard_normal((1, 1, T, NH, HD)).astype(np.float32)
    out = attend(torch, st, Q, [0], [L], T)
    e = rel_err(out[0, 0], expect(oracle, qkv, st, Q[0, 0], K, V, L, T, 0, 0))
    assert e <= TOL, e
    for t in (0, 5, 7):
        o1 = attend(torch, st, Q[:, :, t:t + 1], [0], [L - T + t + 1], 1)
        assert np.array_equal(o1[:, :, 0], out[:, :, t]), t


def test_cfg5_paged_sequences(qkv, oracle, torch_gpu):
    """4 sequences {23,000; 23,000; 60,000; 262,144} in one call, 256-position pages under a seeded permutation,
    preset F with the 2,048 window: each sequence against the oracle; the 60,000 one equals a contiguous store."""
    torch = torch_gpu
    lens, page, win, spec = [23000, 23000, 60000, 262144], 256, 2048, "K*=5r,V*=6"
    print(f"cfg5 lens={lens}", flush=True)
    npg = [-(-L // page) for L in lens]
    st = qkv.KVStore(spec, win=win, n_layers=1, n_seq=4, ctx=max(lens), page=page, n_pages=sum(npg))
    perm = np.random.default_rng(5).permutation(sum(npg))
    o = 0
    for s, L in enumerate(lens):
        st.set_pages(s, perm[o:o + npg[s]])
        o += npg[s]
    rng = np.random.default_rng(50)
    Q = rng.standard_normal((1, 4, 1, NH, HD)).astype(np.float32)
    kv = []
    for s, L in enumerate(lens):
        K, V = f16_kv(rng, L, 1, outliers=True)
        append_all(torch, st, s, K, V, chunks=[16384] * 17, f16=True)
        kv.append((K, V))
    outs = attend(torch, st, Q, [0, 1, 2, 3], lens, 1)
    for s, L in enumerate(lens):
        K, V = kv[s]
        e = rel_err(outs[0, s], expect(oracle, qkv, st, Q[0, s], K, V, L, 1, 0, win))
        assert e <= TOL, (s, L, e)
        if L == 60000:
            flat = qkv.KVStore(spec, win=win, n_layers=1, ctx=L)
            append_all(torch, flat, 0, K, V, chunks=[16384] * 4, f16=True)
            assert np.array_equal(attend(torch, flat, Q[:, s:s + 1], [0], [L], 1)[:, 0], outs[:, s])


def test_cfg2_append_workload(qkv, oracle, torch_gpu):
    """16 layers x 512 steps x 8 fp16 positions into K5r/V6 with the 2,048 window (eviction from step 404 on): every
    main and ring row of layers 0 and 15 read back and compared with the oracle; every layer through the digest."""
    torch = torch_gpu
    nl, steps, win = 16, 512, 2048
    print(f"cfg2 layers={nl} steps={steps}", flush=True)
    L = 8 * steps
    rng = np.random.default_rng(2)
    K, V = f16_kv(rng, L, nl, outliers=True)
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=nl, ctx=L)
    kd = torch.from_numpy(K).half().cuda()
    vd = torch.from_numpy(V).half().cuda()
    for s in range(steps):
        st.append(0, 0, nl, 8 * s, 8, kd[8 * s].data_ptr(), vd[8 * s].data_ptr(), 1)
    torch.cuda.synchronize()
    kvrc = qkv.ring_rows(win)
    rlo = L - kvrc
    head = [0x4d4b444701, L, 0, kvrc, rlo, nl, NKV, 0]
    main_words, ring_words = [], []
    for l in range(nl):
        for w, X, bits, rot in ((0, K, 5, 1), (1, V, 6, 0)):
            for g in range(NKV):
                mq, ms, rq, rs = oracle.store_rows(X[:, l, g], rot, bits, ring=True, threads=8)
                main_words += [oracle.row_digest(mq[p], bits, ms[p]) for p in range(L)]
                ring_words += [oracle.row_digest(rq[p], 8, rs[p]) for p in range(rlo, L)]
                if l in (0, nl - 1):
                    q, sc = st.read_rows(0, l, w, g, 0, L)
                    assert np.array_equal(q, mq) and np.array_equal(sc, ms), (l, w, g)
                    q, sc = st.read_rows(0, l, w, g, rlo, kvrc, ring=True)
                    assert np.array_equal(q, rq[rlo:]) and np.array_equal(sc, rs[rlo:]), (l, w, g)
    assert st.digest(0) == head + main_words + ring_words


def crafted_case(L, T, nl_seed):
    """Q, K, V of one layer whose scores step up and down by 6 log2 units between 32-position tiles: K[p] = noise +
    c(tile) u, Q = 8 u + noise (u a unit vector per kv head), c drawn from {0, 8.3, 16.6, 25} per tile.  Tiles whose
    level exceeds a wave's running maximum by more than 8 log2 units force the O * alpha rescale; the top level recurs
    in every segment, so every segment carries weight into the combine."""
    rng = np.random.default_rng(nl_seed)
    K, V = synth_kv(rng, L, 1)
    ntile = -(-L // 32)
    lev = rng.integers(0, 4, ntile) * 8.3
    Q = np.zeros((1, 1, T, NH, HD), np.float32)
    for g in range(NKV):
        u = rng.standard_normal(HD)
        u = (u / np.linalg.norm(u)).astype(np.float32)
        K[:, 0, g] += np.repeat(lev, 32)[:L, None].astype(np.float32) * u[None]
        Q[0, 0, :, GQA * g:GQA * (g + 1)] = 8 * u + 0.5 * rng.standard_normal((T, GQA, HD)).astype(np.float32)
    return Q, K, V


@pytest.mark.parametrize("L,T,win", [(16385, 1, 2048), (20000, 1, 2048), (20000, 8, 2048), (40000, 2, 640)])
def test_multi_tile_rescale(qkv, oracle, torch_gpu, L, T, win):
    """Contexts above 16,384 (two or more tiles per wave) with crafted score levels that force the online-softmax
    rescale in later tiles; at 20,000 with the 2,048 window, segment 67 (17,152 .. 17,407) holds packed tiles and, from
    the window start 17,280, ring tiles, so waves 0-3 of it each switch from a packed tile to a ring tile."""
    torch = torch_gpu
    print(f"rescale L={L} T={T} win={win}", flush=True)
    Q, K, V = crafted_case(L, T, 60 + L % 97 + T)
    st = qkv.KVStore("K*=5r,V*=6", win=win, n_layers=1, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[4096] * 10)
    out = attend(torch, st, Q, [0], [L], T)
    ref = expect(oracle, qkv, st, Q[0, 0], K, V, L, T, 0, win)
    e = rel_err(out[0, 0], ref)
    assert e <= TOL, e
    assert rescales(oracle, qkv, st, Q[0, 0, T - 1, 0], K[:, 0, 0], L, win) > 0


def rescales(oracle, qkv, st, q, K, L, win):
    """How many tiles raise a wave's running maximum by more than 8 log2 units after its first visible tile, for one
    query row of kv head 0 (the decode kernel: segments of seg_len(L), wave w taking tiles w, w + 4, ..)."""
    from kvcase import expected_kv
    Kd = expected_kv(oracle, K[:L], st.krot[0], st.kbits[0], qkv.window_start(L, win), win > 0)
    s = Kd.astype(np.float64) @ oracle.q_prep(q, st.krot[0]).astype(np.float64) * np.log2(np.e)
    lb = -(-L // 640) * 640
    seg = 128 * -(-lb // 16384)
    n = 0
    for c0 in range(0, L, seg):
        tiles = [s[p:min(p + 32, c0 + seg, L)].max() for p in range(c0, min(c0 + seg, L), 32)]
        for w in range(4):
            m = -np.inf
            for t in tiles[w::4]:
                if m > -np.inf and t > m + 8:
                    n += 1
                if t > m + 8 or m == -np.inf:
                    m = t
    return n
