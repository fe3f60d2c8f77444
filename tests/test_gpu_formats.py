"""Long-context parity over the reference's format matrix (bench/kvattn_bench.cu:398-400: F, D, 44, 76, 85, 58, 66,
47, plus E = K6r/V4r), each against the oracle within 2e-3 relative (max-abs).

Every (K bits, V bits) pair is its own instantiation of the decode kernels, so each format here runs its own
multi-tile code: at 40,013 positions (bucket 40,320, segments of 384 positions, 3 tiles per wave) a wave streams
several tiles of its segment, rescales against a finite running maximum and, with a window, switches from packed to
ring tiles in the segment holding the window start.  One store per format serves every T (the T query tokens are the
store's last T positions):
  T = 1 through the one-group kernel at two and at three workgroups per CU (the small-stage kernel where the format
        has one; the two must be equal bitwise);
  T = 2, 3 and 4 through the 16- and 24-row kernels;
  T = 5 and 8 through the default verify form and through the other one (k_verify / two 24-row batches), bitwise
        equal; at T = 8 tokens 0 and 5 bitwise equal to one-token calls at their own lengths.
(T = 1, 2, 3, 4, 5, 8: the reference's own T set for this matrix.)
One case at 200,031 positions (bucket 200,320, 13 tiles per wave) runs D at T = 1 and 8.  The prefill kernel of each
format (k_prefill3, one instantiation per (K bits, V bits) pair as well) runs a 2,600-position prompt.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from kvcase import GQA, HD, NH, NKV, append_all, expected_attention, expected_kv, rel_err, synth_kv

pytestmark = pytest.mark.gpu
TOL = 2e-3

# name, spec, window (the reference's Fmt{kb, vb, kr, win}: kr rotates K)
FORMATS = [
    ("F", "K*=5r,V*=5", 2048),
    ("D", "K*=6,V*=5", 2048),
    ("E", "K*=6r,V*=4r", 2048),
    ("44", "K*=4,V*=4", 2048),
    ("76", "K*=7,V*=6", 0),
    ("85", "K*=8,V*=5", 2048),
    ("58", "K*=5r,V*=8", 2048),
    ("66", "K*=6r,V*=6", 0),
    ("66vr", "K*=6r,V*=6r", 0),
    ("47", "K*=4,V*=7", 2048),
]


def _store(qkv, torch, spec, win, L, seed):
    rng = np.random.default_rng(seed)
    K, V = synth_kv(rng, L, 1, outliers=True)
    K = K.astype(np.float16).astype(np.float32)
    V = V.astype(np.float16).astype(np.float32)
    st = qkv.KVStore(spec, win=win, n_layers=1, ctx=L)
    append_all(torch, st, 0, K, V, chunks=[16384] * (L // 16384 + 1), f16=True)
    return rng, st, K, V


def _operands(oracle, qkv, st, K, V, L, win):
    """The fp16 operands of every kv head, dequantized once: [4][L][256] for K and V."""
    ws = qkv.window_start(L, win)
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    Kd = np.stack([expected_kv(oracle, K[:, 0, g], kr, kb, ws, win > 0 and kb != 8) for g in range(NKV)])
    Vd = np.stack([expected_kv(oracle, V[:, 0, g], vr, vb, ws, win > 0 and vb != 8) for g in range(NKV)])
    return Kd, Vd


def _expected(oracle, st, Q, Kd, Vd, T):
    """Q [T][24][256] -> [T][24][256]: fp64 attention per kv head on the dequantized operands (the oracle's threads)."""
    R = GQA * T
    q = np.zeros((NKV, R, HD), np.float32)
    for g in range(NKV):
        for r in range(R):
            q[g, r] = oracle.q_prep(Q[r % T, GQA * g + r // T], st.krot[0])
    out = np.zeros((T, NH, HD), np.float32)
    with ThreadPoolExecutor(NKV) as ex:
        ys = list(ex.map(lambda g: oracle.attn_exact(q[g], Kd[g], Vd[g], T), range(NKV)))
    for g, y in enumerate(ys):
        for r in range(R):
            v = oracle.fwht(y[r]) if st.vrot[0] else y[r]
            out[r % T, GQA * g + r // T] = v
    return out


def _attend(torch, st, Q, L, T):
    q = torch.from_numpy(np.ascontiguousarray(Q[None, None], np.float32)).cuda()
    out = torch.full_like(q, float("nan"))
    st.attend(0, 1, [0], [L], T, q.data_ptr(), out.data_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy()[0, 0]


@pytest.mark.parametrize("name,spec,win", FORMATS, ids=[f[0] for f in FORMATS])
def test_format_long_context(qkv, oracle, torch_gpu, name, spec, win):
    torch = torch_gpu
    L = 40013
    print(f"format {name} ({spec}, win {win}) L={L}", flush=True)
    rng, st, K, V = _store(qkv, torch, spec, win, L, 400 + len(name) * 7 + int(name.isdigit()) * 31 + win % 7)
    Kd, Vd = _operands(oracle, qkv, st, K, V, L, win)
    for T in (1, 2, 3, 4, 5, 8):
        Q = rng.standard_normal((T, NH, HD)).astype(np.float32)
        out = _attend(torch, st, Q, L, T)
        e = rel_err(out, _expected(oracle, st, Q, Kd, Vd, T))
        assert e <= TOL, (name, T, e)
        if T == 1:
            for occ in (2, 3):
                st.config("occupancy", occ)
                assert np.array_equal(_attend(torch, st, Q, L, T), out), (name, "occupancy", occ)
            st.config("occupancy", 0)
        if T >= 5:
            for wide in (0, 1):
                st.config("wide", wide)
                assert np.array_equal(_attend(torch, st, Q, L, T), out), (name, "wide", wide)
            st.config("wide", 2)
        if T == 8:
            # T-invariance (bench/dattn_bench.cu:1140-1160): token t equals a one-token call at its own length
            for t in (0, 5):
                o1 = _attend(torch, st, Q[t:t + 1], L - T + t + 1, 1)
                assert np.array_equal(o1[0], out[t]), (name, "token", t)


def test_format_d_200031(qkv, oracle, torch_gpu):
    """D (K6/V5, window 2,048) at 200,031 positions: 13 tiles per wave, T = 1 at both occupancies and T = 8."""
    torch = torch_gpu
    L, spec, win = 200031, "K*=6,V*=5", 2048
    print(f"format D L={L}", flush=True)
    rng, st, K, V = _store(qkv, torch, spec, win, L, 431)
    Kd, Vd = _operands(oracle, qkv, st, K, V, L, win)
    del K, V
    for T in (1, 8):
        Q = rng.standard_normal((T, NH, HD)).astype(np.float32)
        out = _attend(torch, st, Q, L, T)
        e = rel_err(out, _expected(oracle, st, Q, Kd, Vd, T))
        assert e <= TOL, (T, e)
        if T == 1:
            st.config("occupancy", 3)
            assert np.array_equal(_attend(torch, st, Q, L, T), out)
            st.config("occupancy", 0)


@pytest.mark.parametrize("name,spec,win", FORMATS, ids=[f[0] for f in FORMATS])
def test_format_prefill(qkv, oracle, torch_gpu, name, spec, win):
    """The prefill kernel of each format (its own (K bits, V bits) instantiation): a 2,600-position prompt in two chunks
    over five 640-position pieces (packed rows below the window start, ring rows from it), the first and the last piece
    against the oracle within 2e-3, and the same prompt in one chunk bitwise equal."""
    from test_gpu_prefill import pieces, run_prefill

    torch = torch_gpu
    rng = np.random.default_rng(900 + len(name) * 3 + win % 11)
    P = 2600
    K, V = synth_kv(rng, P, 1, outliers=True)
    Q = rng.standard_normal((1, P, NH, HD)).astype(np.float32)
    st, out = run_prefill(qkv, torch, spec, win, K, V, Q, [1300, 1300], P)
    kb, vb, kr, vr = st.kbits[0], st.vbits[0], st.krot[0], st.vrot[0]
    for a, b in (pieces(P)[0], pieces(P)[-1]):
        ws = qkv.window_start(b, win)
        ref = expected_attention(oracle, Q[0, a:b], K[:b, 0], V[:b, 0], b - a, kr, vr, kb, vb, ws, win > 0 and kb != 8,
                                 win > 0 and vb != 8)
        e = rel_err(out[0, a:b], ref)
        assert e <= TOL, (name, a, b, e)
    st.close()
    st2, out2 = run_prefill(qkv, torch, spec, win, K, V, Q, [P], P)
    assert np.array_equal(out2, out), name
    st2.close()
