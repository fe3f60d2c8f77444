"""ctypes wrapper of the CPU oracle (kv_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker
and the host-core baseline.  The product library never uses it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libkv_oracle.so")
HD = 256

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            from . import build as _b  # noqa: F401  (package import when available)
        l = ctypes.CDLL(LIB)
        vp, ci, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "kvo_f2h": (ctypes.c_uint16, [cf]),
            "kvo_h2f": (cf, [ctypes.c_uint16]),
            "kvo_store_q8": (None, [vp, vp, vp]),
            "kvo_store_qn": (None, [vp, vp, vp, ci]),
            "kvo_fwht256": (None, [vp]),
            "kvo_codes": (None, [vp, ci, vp]),
            "kvo_dequant_f32": (None, [vp, vp, ci, vp]),
            "kvo_dequant_f16": (None, [vp, vp, ci, vp]),
            "kvo_dequant_rows": (None, [vp, vp, ci, ci, vp, ci]),
            "kvo_store_row": (None, [vp, ci, ci, vp, vp, vp, vp]),
            "kvo_ring_refill_row": (None, [vp, vp, ci, vp, vp]),
            "kvo_ws": (ci, [ci, ci]),
            "kvo_kvrc": (ci, [ci]),
            "kvo_cap_T": (ci, [ci, ci]),
            "kvo_q_prep": (None, [vp, ci, vp]),
            "kvo_attn_exact": (None, [vp, vp, vp, ci, ci, ci, vp]),
            "kvo_attn_chunked": (ci, [vp, vp, vp, ci, ci, ci, vp, ci]),
            "kvo_attn_heads": (ci, [vp, vp, vp, ci, ci, ci, ci, vp, ci]),
            "kvo_store_rows": (None, [vp, ci, ci, ci, vp, vp, vp, vp, ci]),
            "kvo_dg_hash": (ctypes.c_uint64, [vp, ctypes.c_size_t, ctypes.c_uint64]),
            "kvo_gate": (cf, [cf, cf]),
            "kvo_q32_row": (None, [vp, vp, vp, vp]),
            "kvo_rope_rows": (None, [ci, ci, vp]),
            "kvo_qk_prep": (None, [vp, vp, vp, vp]),
            "kvo_row_digest": (ctypes.c_uint64, [vp, ci, vp]),
            "kvo_now": (ctypes.c_double, []),
        }
        for n, (r, a) in sig.items():
            f = getattr(l, n)
            f.restype = r
            f.argtypes = a
        _lib = l
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f2h(x):
    return lib().kvo_f2h(float(x))


def h2f(b):
    return lib().kvo_h2f(int(b))


def row_bytes(bits):
    return 32 * bits


def store_q8(v):
    v = np.ascontiguousarray(v, np.float32)
    q = np.zeros(HD, np.int8)
    s = np.zeros(8, np.uint16)
    lib().kvo_store_q8(_p(v), _p(q), _p(s))
    return q, s


def store_qn(v, bits):
    v = np.ascontiguousarray(v, np.float32)
    q = np.zeros(row_bytes(bits), np.uint8)
    s = np.zeros(8, np.uint16)
    lib().kvo_store_qn(_p(v), _p(q), _p(s), bits)
    return q, s


def store(v, bits):
    """(value bytes as uint8, scales) of one row in `bits` (8: q8)."""
    if bits == 8:
        q, s = store_q8(v)
        return q.view(np.uint8), s
    return store_qn(v, bits)


def fwht(v):
    v = np.array(v, np.float32, copy=True)
    lib().kvo_fwht256(_p(v))
    return v


def codes(q, bits):
    q = np.ascontiguousarray(q).view(np.uint8)
    out = np.zeros(HD, np.int32)
    lib().kvo_codes(_p(q), bits, _p(out))
    return out


def dequant(q, s, bits, f16=False):
    q = np.ascontiguousarray(q).view(np.uint8)
    s = np.ascontiguousarray(s, np.uint16)
    out = np.zeros(HD, np.float32)
    (lib().kvo_dequant_f16 if f16 else lib().kvo_dequant_f32)(_p(q), _p(s), bits, _p(out))
    return out


def dequant_rows(q, s, bits, f16=True):
    """rows [n][rb] bytes + scales [n][8] -> fp32 [n][256]"""
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.uint16)
    n = q.shape[0]
    out = np.zeros((n, HD), np.float32)
    lib().kvo_dequant_rows(_p(q), _p(s), bits, n, _p(out), int(f16))
    return out


def store_row(v, rotate, bits, ring=True):
    """kv_store: (main bytes, main scales, ring bytes or None, ring scales or None)."""
    v = np.ascontiguousarray(v, np.float32)
    mq = np.zeros(row_bytes(bits), np.uint8)
    ms = np.zeros(8, np.uint16)
    rq = np.zeros(HD, np.int8) if ring else None
    rs = np.zeros(8, np.uint16) if ring else None
    lib().kvo_store_row(_p(v), int(rotate), bits, _p(mq), _p(ms), _p(rq) if ring else None, _p(rs) if ring else None)
    return mq, ms, (rq.view(np.uint8) if ring else None), rs


def store_rows(x, rot, bits, ring=True, threads=1):
    """Rows [n][256] -> (main [n][rb], scales [n][8], ring [n][256], ring scales [n][8])."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[0]
    mq = np.zeros((n, row_bytes(bits)), np.uint8)
    ms = np.zeros((n, 8), np.uint16)
    rq = np.zeros((n, HD), np.int8) if ring else None
    rs = np.zeros((n, 8), np.uint16) if ring else None
    lib().kvo_store_rows(_p(x), n, int(rot), bits, _p(mq), _p(ms), _p(rq) if ring else None, _p(rs) if ring else None, threads)
    return mq, ms, (rq.view(np.uint8) if ring else None), rs


def ring_refill_row(mq, ms, bits):
    mq = np.ascontiguousarray(mq, np.uint8)
    ms = np.ascontiguousarray(ms, np.uint16)
    rq = np.zeros(HD, np.int8)
    rs = np.zeros(8, np.uint16)
    lib().kvo_ring_refill_row(_p(mq), _p(ms), bits, _p(rq), _p(rs))
    return rq.view(np.uint8), rs


def ws(L, win):
    return lib().kvo_ws(L, win)


def kvrc(win):
    return lib().kvo_kvrc(win)


def cap_T(n, T):
    return lib().kvo_cap_T(n, T)


def q_prep(q, rotate):
    q = np.ascontiguousarray(q, np.float32)
    out = np.zeros(HD, np.float32)
    lib().kvo_q_prep(_p(q), int(rotate), _p(out))
    return out


def attn_exact(q, K, V, T):
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    R, L = q.shape[0], K.shape[0]
    out = np.zeros((R, HD), np.float32)
    lib().kvo_attn_exact(_p(q), _p(K), _p(V), L, T, R, _p(out))
    return out


def attn_chunked(q, K, V, T, threads=1):
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    R, L = q.shape[0], K.shape[0]
    out = np.zeros((R, HD), np.float32)
    r = lib().kvo_attn_chunked(_p(q), _p(K), _p(V), L, T, R, _p(out), threads)
    assert r == 0
    return out


def attn_heads(q, K, V, T, threads):
    """q [nkv][R][256], K/V [nkv][L][256] -> [nkv][R][256] (the reference's split-K arithmetic per head)."""
    q = np.ascontiguousarray(q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    nkv, R, _ = q.shape
    L = K.shape[1]
    out = np.zeros((nkv, R, HD), np.float32)
    r = lib().kvo_attn_heads(_p(q), _p(K), _p(V), nkv, L, T, R, _p(out), threads)
    assert r == 0
    return out


def dg_hash(b, seed=0xcbf29ce484222325):
    b = np.ascontiguousarray(b).view(np.uint8)
    return lib().kvo_dg_hash(_p(b), b.size, seed)


def row_digest(q, bits, s):
    q = np.ascontiguousarray(q).view(np.uint8)
    s = np.ascontiguousarray(s, np.uint16)
    return lib().kvo_row_digest(_p(q), bits, _p(s))


def now():
    return lib().kvo_now()


def gate(y, g):
    y = np.ascontiguousarray(y, np.float32).ravel()
    g = np.ascontiguousarray(g, np.float32).ravel()
    return np.array([lib().kvo_gate(float(a), float(b)) for a, b in zip(y, g)], np.float32)


def q32_row(o):
    """One token's output row o [24 * 256] -> (xa [192][16] int8, xb [192][16] int8, meta [192][4] uint16)."""
    o = np.ascontiguousarray(o, np.float32).ravel()
    assert o.size == 24 * HD
    xa = np.zeros((192, 16), np.int8)
    xb = np.zeros((192, 16), np.int8)
    meta = np.zeros((192, 4), np.uint16)
    lib().kvo_q32_row(_p(o), _p(xa), _p(xb), _p(meta))
    return xa, xb, meta


def rope_rows(p0, n):
    """RoPE text table rows p0 .. p0+n-1 -> float32 [n][32][2] (cos, sin)."""
    out = np.zeros((n, 32, 2), np.float32)
    lib().kvo_rope_rows(p0, n, _p(out))
    return out


def qk_prep(x, w, rc):
    """RMSNorm (weights w [256]) + RoPE (table row rc [32][2]) of one row x [256], in the HIP kernels' order."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rc = np.ascontiguousarray(rc, np.float32)
    assert x.size == HD and w.size == HD and rc.size == 64
    out = np.zeros(HD, np.float32)
    lib().kvo_qk_prep(_p(x), _p(w), _p(rc), _p(out))
    return out
