"""A seeded randomized sweep over the store and attention parameters: per case a random MK_KV spec (bits 4..8 per side,
rotations), window, context length, T (capped to one 640-bucket as the reference's att_cap_T does), 1..3 sequences
on a shared page pool with a shuffled page table, the decode occupancy knob, a capped grid and an L2 prefetch of the
call on a second stream.  Every stored row is compared bit for bit and every attention
output within 2e-3 (max-abs relative) against the oracle.  QKV_SWEEP_CASES sets the number of cases (default 8);
QKV_SWEEP_LONG_CASES the number of long-context cases (default 4), QKV_SWEEP_PREFILL_CASES the number of prefill cases
(default 4)."""
import os

import numpy as np
import pytest

from kvcase import HD, NH, NKV, check_rows, expected_attention, rel_err, synth_kv

pytestmark = pytest.mark.gpu


def random_spec(rng):
    items = []
    for side in "KV":
        b = int(rng.integers(4, 9))
        items.append(f"{side}*={b}{'r' if b < 8 and rng.random() < 0.5 else ''}")
    return ",".join(items)


@pytest.mark.parametrize("case", range(int(os.environ.get("QKV_SWEEP_CASES", "8"))))
def test_random_case(qkv, oracle, torch_gpu, case):
    torch = torch_gpu
    rng = np.random.default_rng(1000 + case)
    spec = random_spec(rng)
    win = int(rng.choice([0, 256, 640, 2048]))
    n_seq = int(rng.integers(1, 4))
    page = 256
    lens = [int(rng.integers(1, 4200)) for _ in range(n_seq)]
    ctx = 4352
    npg = ctx // page
    T = int(rng.integers(1, 9))
    T = min(T, min(lens))
    T = min([qkv.cap_T(L - T, T) for L in lens] + [T])  # the T rows of every sequence stay inside one bucket
    T = max(T, 1)
    st = qkv.KVStore(spec, win=win, n_layers=1, n_seq=n_seq, ctx=ctx, page=page, n_pages=n_seq * npg)
    knobs = np.random.default_rng(5000 + case)
    occ = int(knobs.choice([0, 3]))  # 3: small stages where the format allows
    st.config("occupancy", occ)
    max_blocks = int(knobs.choice([0, 0, 1, 37, 255]))
    st.config("max_blocks", max_blocks)
    prefetch = bool(knobs.random() < 0.4)
    perm = rng.permutation(n_seq * npg)
    data = []
    print(f"case {case}: spec={spec} win={win} lens={lens} T={T} occupancy={occ} max_blocks={max_blocks} prefetch={prefetch}", flush=True)
    for s, L in enumerate(lens):
        st.set_pages(s, perm[s * npg:(s + 1) * npg])
        K, V = synth_kv(rng, L, 1, outliers=bool(rng.random() < 0.5))
        k = torch.from_numpy(K).cuda()
        v = torch.from_numpy(V).cuda()
        st.append(s, 0, 1, 0, L, k.data_ptr(), v.data_ptr(), 0)
        torch.cuda.synchronize()
        check_rows(oracle, st, K, V, seq=s, ring_from=max(0, L - qkv.ring_rows(win)) if win else 0)
        data.append((K, V))
    Q = rng.standard_normal((1, n_seq, T, NH, HD)).astype(np.float32)
    q = torch.from_numpy(Q).cuda()
    o = torch.full_like(q, float("nan"))
    if prefetch:
        side = torch.cuda.Stream()
        st.prefetch(0, 1, list(range(n_seq)), lens, T, int(knobs.integers(1, 5)), side.cuda_stream)
        side.synchronize()
    st.attend(0, 1, list(range(n_seq)), lens, T, q.data_ptr(), o.data_ptr())
    torch.cuda.synchronize()
    out = o.cpu().numpy()
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    for s, L in enumerate(lens):
        K, V = data[s]
        ws = qkv.window_start(L, win)
        ref = expected_attention(oracle, Q[0, s], K[:, 0], V[:, 0], T, kr, vr, kb, vb, ws, win > 0 and kb != 8, win > 0 and vb != 8)
        assert rel_err(out[0, s], ref) <= 2e-3, (case, spec, win, L, T)
    st.close()


@pytest.mark.parametrize("case", range(int(os.environ.get("QKV_SWEEP_LONG_CASES", "4"))))
def test_random_long_case(qkv, oracle, torch_gpu, case):
    """The same sweep at long contexts (16,385 .. 70,000 positions: several tiles per wave, the window start inside a
    segment), 1..2 paged sequences, and the verify form knob at T >= 5 (the forms give the same bits, so any may run), a capped grid and a prefetch of the call."""
    torch = torch_gpu
    rng = np.random.default_rng(7000 + case)
    spec = random_spec(rng)
    win = int(rng.choice([0, 640, 2048]))
    n_seq = int(rng.integers(1, 3))
    page = 256
    lens = [int(rng.integers(16385, 70001)) for _ in range(n_seq)]
    ctx = max(lens) + page
    npg = -(-ctx // page)
    T = int(rng.integers(1, 9))
    T = min([qkv.cap_T(L - T, T) for L in lens] + [T])
    T = max(T, 1)
    st = qkv.KVStore(spec, win=win, n_layers=1, n_seq=n_seq, ctx=ctx, page=page, n_pages=n_seq * npg)
    occ = int(rng.choice([0, 2, 3]))
    wide = int(rng.choice([0, 1, 2]))
    st.config("occupancy", occ)
    st.config("wide", wide)
    knobs = np.random.default_rng(9000 + case)
    max_blocks = int(knobs.choice([0, 0, 7, 300]))
    st.config("max_blocks", max_blocks)
    prefetch = bool(knobs.random() < 0.5)
    perm = rng.permutation(n_seq * npg)
    data = []
    print(f"long case {case}: spec={spec} win={win} lens={lens} T={T} occupancy={occ} wide={wide} max_blocks={max_blocks} "
          f"prefetch={prefetch}", flush=True)
    for s, L in enumerate(lens):
        st.set_pages(s, perm[s * npg:(s + 1) * npg])
        K, V = synth_kv(rng, L, 1, outliers=bool(rng.random() < 0.5))
        K = K.astype(np.float16).astype(np.float32)
        V = V.astype(np.float16).astype(np.float32)
        for p in range(0, L, 16384):
            k = torch.from_numpy(K[p:p + 16384]).half().cuda()
            v = torch.from_numpy(V[p:p + 16384]).half().cuda()
            st.append(s, 0, 1, p, k.shape[0], k.data_ptr(), v.data_ptr(), 1)
        torch.cuda.synchronize()
        data.append((K, V))
    Q = rng.standard_normal((1, n_seq, T, NH, HD)).astype(np.float32)
    q = torch.from_numpy(Q).cuda()
    o = torch.full_like(q, float("nan"))
    if prefetch:
        side = torch.cuda.Stream()
        st.prefetch(0, 1, list(range(n_seq)), lens, T, int(knobs.integers(1, 9)), side.cuda_stream)
        side.synchronize()
    st.attend(0, 1, list(range(n_seq)), lens, T, q.data_ptr(), o.data_ptr())
    torch.cuda.synchronize()
    out = o.cpu().numpy()
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    for s, L in enumerate(lens):
        K, V = data[s]
        ws = qkv.window_start(L, win)
        ref = expected_attention(oracle, Q[0, s], K[:, 0], V[:, 0], T, kr, vr, kb, vb, ws, win > 0 and kb != 8, win > 0 and vb != 8)
        assert rel_err(out[0, s], ref) <= 2e-3, (case, spec, win, L, T)
    st.close()


@pytest.mark.parametrize("case", range(int(os.environ.get("QKV_SWEEP_PREFILL_CASES", "4"))))
def test_random_prefill_case(qkv, oracle, torch_gpu, case):
    """Prefill under the same kind of draw: a random spec and window, 1 or 2 layers, a prompt of 1 .. 3,500 positions in
    1 .. 4 random chunks, contiguous or on a permuted page pool.  The first and last 640-position pieces against the
    oracle within 2e-3, the whole prompt in one chunk on a fresh store bitwise equal, the stored rows bit-exact."""
    from test_gpu_prefill import pieces, run_prefill

    torch = torch_gpu
    rng = np.random.default_rng(11000 + case)
    spec = random_spec(rng)
    win = int(rng.choice([0, 256, 640, 2048]))
    nl = int(rng.integers(1, 3))
    P = int(rng.integers(1, 3501))
    cuts = sorted(set(int(x) for x in rng.integers(1, P, size=int(rng.integers(0, 4))))) if P > 1 else []
    chunks = [b - a for a, b in zip([0] + cuts, cuts + [P])]
    paged = bool(rng.random() < 0.5)
    print(f"prefill case {case}: spec={spec} win={win} nl={nl} P={P} chunks={chunks} paged={paged}", flush=True)
    K, V = synth_kv(rng, P, nl, outliers=bool(rng.random() < 0.5))
    Q = rng.standard_normal((nl, P, NH, HD)).astype(np.float32)
    if paged:
        page, ctx = 256, 3584
        npg = ctx // page
        st = qkv.KVStore(spec, win=win, n_layers=nl, n_seq=2, ctx=ctx, page=page, n_pages=2 * npg)
        st.set_pages(1, rng.permutation(2 * npg)[:npg])
        outs, p = [], 0
        for c in chunks:
            k = torch.from_numpy(np.ascontiguousarray(K[p:p + c])).cuda()
            v = torch.from_numpy(np.ascontiguousarray(V[p:p + c])).cuda()
            q = torch.from_numpy(np.ascontiguousarray(Q[:, p:p + c])).cuda()
            o = torch.empty_like(q)
            st.prefill(1, 0, nl, p, c, k.data_ptr(), v.data_ptr(), 0, q.data_ptr(), o.data_ptr())
            torch.cuda.synchronize()
            outs.append(o.cpu().numpy())
            p += c
        out = np.concatenate(outs, axis=1)
        check_rows(oracle, st, K, V, seq=1, ring_from=max(0, P - qkv.ring_rows(win)) if win else 0)
    else:
        st, out = run_prefill(qkv, torch, spec, win, K, V, Q, chunks, P)
        check_rows(oracle, st, K, V, ring_from=max(0, P - qkv.ring_rows(win)) if win else 0)
    for l in range(nl):
        kb, vb, kr, vr = st.kbits[l], st.vbits[l], st.krot[l], st.vrot[l]
        for a, b in {pieces(P)[0], pieces(P)[-1]}:
            ws = qkv.window_start(b, win)
            ref = expected_attention(oracle, Q[l, a:b], K[:b, l], V[:b, l], b - a, kr, vr, kb, vb, ws, win > 0 and kb != 8,
                                     win > 0 and vb != 8)
            assert rel_err(out[l, a:b], ref) <= 2e-3, (case, spec, win, l, a, b)
    st.close()
    st2, out2 = run_prefill(qkv, torch, spec, win, K, V, Q, [P], P)
    assert np.array_equal(out2, out), case
    st2.close()
