"""ctypes binding of the KV-path C ABI (include/qwen38_kv.h), in the style of the reference's server/mk_engine.py
argtypes tables (server/mk_engine.py:13-100).  It is a thin host-side mirror: every call goes straight to
libqwen38_kv.so, which runs the HIP kernels; there is no Python or CPU compute path.

Device buffers are passed as integer device addresses (e.g. torch.Tensor.data_ptr() of a CUDA tensor) and a stream
handle (torch.cuda.current_stream().cuda_stream, or 0 for the default stream).
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QKV_LIB") or os.path.join(HERE, "libqwen38_kv.so")

NKV, NH, HD = 4, 24, 256

_c_int, _c_ll, _c_vp, _c_cp = ctypes.c_int, ctypes.c_longlong, ctypes.c_void_p, ctypes.c_char_p
_P_int = ctypes.POINTER(ctypes.c_int)
_P_ll = ctypes.POINTER(ctypes.c_longlong)
_P_u64 = ctypes.POINTER(ctypes.c_ulonglong)
_P_u16 = ctypes.POINTER(ctypes.c_ushort)

# name -> (restype, argtypes): the exports of include/qwen38_kv.h
SIGNATURES = {
    "mk_last_error": (_c_cp, []),
    "mk_kv_new": (_c_vp, [_c_cp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "mk_free": (None, [_c_vp]),
    "mk_kv_set_pages": (_c_int, [_c_vp, _c_int, _P_int, _c_int]),
    "mk_kv_append": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_int, _c_vp]),
    "mk_kv_attend": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _P_int, _P_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "mk_kv_prefetch": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _P_int, _P_int, _c_int, _c_int, _c_vp]),
    "mk_kv_append_attend": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _P_int, _P_int, _c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_vp]),
    "mk_kv_attend_noalloc": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _P_int, _P_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "mk_kv_attend_gated": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _P_int, _P_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _P_u16,
                                    _c_vp]),
    "mk_kv_set_rope": (_c_int, [_c_vp, _c_vp, _c_int]),
    "mk_kv_append_prep": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp]),
    "mk_kv_attend_prep": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _P_int, _P_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _P_u16,
                                   _c_vp]),
    "mk_kv_prefill": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_vp]),
    "mk_kv_prefill_prep": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                    _P_u16, _c_vp]),
    "mk_truncate": (_c_int, [_c_vp, _c_int]),
    "mk_rewind_to": (_c_int, [_c_vp, _c_int]),
    "mk_kv_rewind": (_c_int, [_c_vp, _c_int, _c_int]),
    "mk_kv_sizes": (None, [_c_vp, _P_ll, _P_ll, _P_ll, _P_ll]),
    "mk_state_digest": (_c_int, [_c_vp, _P_u64, _c_int]),
    "mk_kv_state_digest": (_c_int, [_c_vp, _c_int, _P_u64, _c_int]),
    "mk_kv_read_rows": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _P_u16]),
    "mk_kv_write_rows": (_c_int, [_c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp, _P_u16]),
    "mk_kv_ring_snapshot": (_c_ll, [_c_vp, _c_int, _c_vp, _c_ll]),
    "mk_kv_ring_restore": (_c_int, [_c_vp, _c_int, _c_int, _c_vp, _c_ll]),
    "mk_kv_config": (_c_int, [_c_vp, _c_cp, _c_ll]),
    "mk_kv_profile": (_c_int, [_c_vp, _c_int, ctypes.POINTER(ctypes.c_double), _c_int]),
    "mk_kv_window_start": (_c_int, [_c_int, _c_int]),
    "mk_kv_ring_rows": (_c_int, [_c_int]),
    "mk_kv_cap_T": (_c_int, [_c_int, _c_int]),
    "mk_kv_parse_spec": (_c_int, [_c_cp, _c_int, _P_int]),
}

_lib = None


class KVError(RuntimeError):
    pass


def lib():
    """Load the native library (raises if it was not built: there is no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise KVError(f"{LIB_PATH} is missing: build it with qwen38-megakernel_amd/build.py")
        try:
            # A process must hold one HIP runtime.  PyTorch ships its own libamdhip64 (soname libamdhip64.so.7, loaded
            # under the file name libamdhip64.so); loading torch first makes this library's libamdhip64.so.7 bind to
            # that copy instead of starting a second runtime that then sees no device.
            import torch  # noqa: F401
        except ImportError:
            pass
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def last_error():
    return lib().mk_last_error().decode()


def _check(r):
    if r < 0:
        raise KVError(last_error())
    return r


def window_start(L, win):
    return lib().mk_kv_window_start(L, win)


def ring_rows(win):
    return lib().mk_kv_ring_rows(win)


def cap_T(n, T):
    return lib().mk_kv_cap_T(n, T)


def parse_spec(spec, n_layers):
    """MK_KV spec -> (K bits, V bits, K rotated, V rotated), each a list of n_layers ints."""
    out = (ctypes.c_int * (4 * n_layers))()
    _check(lib().mk_kv_parse_spec(spec.encode() if spec is not None else None, n_layers, out))
    v = list(out)
    return v[:n_layers], v[n_layers:2 * n_layers], v[2 * n_layers:3 * n_layers], v[3 * n_layers:]


class KVStore:
    """One quantized KV store (mk_kv_new).  Shapes follow include/qwen38_kv.h."""

    def __init__(self, spec="", win=0, n_layers=16, n_seq=1, ctx=4096, page=0, n_pages=0, win_all=0):
        L = lib()
        h = L.mk_kv_new(spec.encode() if spec else None, win, win_all, n_layers, n_seq, ctx, page, n_pages)
        if not h:
            raise KVError(last_error())
        self.h = h
        self.n_layers, self.n_seq, self.ctx, self.win = n_layers, n_seq, ctx, win
        self.kbits, self.vbits, self.krot, self.vrot = parse_spec(spec, n_layers)

    def close(self):
        if self.h:
            lib().mk_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_pages(self, seq, pages):
        arr = (ctypes.c_int * len(pages))(*[int(p) for p in pages])
        _check(lib().mk_kv_set_pages(self.h, seq, arr, len(pages)))

    def append(self, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, dtype, stream=0):
        _check(lib().mk_kv_append(self.h, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, dtype, stream))

    def attend(self, layer0, n_layers, seqs, lens, T, q_ptr, out_ptr, stream=0):
        n = len(seqs)
        s = (ctypes.c_int * n)(*seqs)
        l = (ctypes.c_int * n)(*lens)
        _check(lib().mk_kv_attend(self.h, layer0, n_layers, n, s, l, T, q_ptr, out_ptr, stream))

    def append_attend(self, layer0, n_layers, seqs, lens, T, k_ptr, v_ptr, dtype, q_ptr, out_ptr, stream=0):
        """append of positions lens[i] - T .. lens[i] - 1 ([n_seq][T][n_layers][4][256]) and attend, in one launch."""
        n = len(seqs)
        s = (ctypes.c_int * n)(*seqs)
        l = (ctypes.c_int * n)(*lens)
        _check(lib().mk_kv_append_attend(self.h, layer0, n_layers, n, s, l, T, k_ptr, v_ptr, dtype, q_ptr, out_ptr, stream))

    def prefetch(self, layer0, n_layers, seqs, lens, T, tiles=1, stream=0):
        """read the first `tiles` tiles of each wave slice of a later attend into the L2 its workgroups use."""
        n = len(seqs)
        s = (ctypes.c_int * n)(*seqs)
        l = (ctypes.c_int * n)(*lens)
        _check(lib().mk_kv_prefetch(self.h, layer0, n_layers, n, s, l, T, tiles, stream))

    def attend_noalloc(self, layer0, n_layers, seqs, lens, T, q_ptr, out_ptr, stream=0):
        """attend with the partials in the library's per-device array (mk_kv_attend_noalloc): allocates nothing."""
        n = len(seqs)
        s = (ctypes.c_int * n)(*seqs)
        l = (ctypes.c_int * n)(*lens)
        _check(lib().mk_kv_attend_noalloc(self.h, layer0, n_layers, n, s, l, T, q_ptr, out_ptr, stream))

    def attend_gated(self, layer0, n_layers, seqs, lens, T, q_ptr, gate_ptr, out_ptr, q32a=0, q32b=0, q32meta=0, stream=0):
        """attend + the output gate (+ the int8 o_proj units when q32a / q32b / q32meta are device pointers)."""
        n = len(seqs)
        s = (ctypes.c_int * n)(*seqs)
        l = (ctypes.c_int * n)(*lens)
        _check(lib().mk_kv_attend_gated(self.h, layer0, n_layers, n, s, l, T, q_ptr, gate_ptr, out_ptr, q32a or None, q32b or None,
                                        ctypes.cast(q32meta, _P_u16) if q32meta else None, stream))

    def set_rope(self, table_ptr=0, rows=0):
        """Use a device RoPE table [rows][32] (cos, sin) for the prep calls; 0 = the store's own text table."""
        _check(lib().mk_kv_set_rope(self.h, table_ptr or None, rows))

    def append_prep(self, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, knorm_ptr, stream=0):
        """append of raw fp32 K rows: RMSNorm (k_norm weights) + RoPE inside the append kernel."""
        _check(lib().mk_kv_append_prep(self.h, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, knorm_ptr, stream))

    def attend_prep(self, layer0, n_layers, seqs, lens, T, qg_ptr, qnorm_ptr, out_ptr, q32a=0, q32b=0, q32meta=0, stream=0):
        """attend_gated on the raw q_proj output [..][24][q 256 | gate 256]: q-norm + RoPE, attention, gate."""
        n = len(seqs)
        s = (ctypes.c_int * n)(*seqs)
        l = (ctypes.c_int * n)(*lens)
        _check(lib().mk_kv_attend_prep(self.h, layer0, n_layers, n, s, l, T, qg_ptr, qnorm_ptr, out_ptr, q32a or None, q32b or None,
                                       ctypes.cast(q32meta, _P_u16) if q32meta else None, stream))

    def prefill(self, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, dtype, q_ptr, out_ptr, stream=0):
        """Store K/V of positions pos .. pos+T-1 and attend the chunk's queries causally (640-bucket pieces)."""
        _check(lib().mk_kv_prefill(self.h, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, dtype, q_ptr, out_ptr, stream))

    def prefill_prep(self, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, knorm_ptr, qg_ptr, qnorm_ptr, out_ptr, q32a=0, q32b=0, q32meta=0,
                     stream=0):
        """prefill on raw projections: K/Q prep, attention, gate (+ the int8 o_proj units)."""
        _check(lib().mk_kv_prefill_prep(self.h, seq, layer0, n_layers, pos, T, k_ptr, v_ptr, knorm_ptr, qg_ptr, qnorm_ptr, out_ptr,
                                        q32a or None, q32b or None, ctypes.cast(q32meta, _P_u16) if q32meta else None, stream))

    def rewind(self, seq, pos):
        _check(lib().mk_kv_rewind(self.h, seq, pos))

    def sizes(self):
        a, b, c, d = ctypes.c_longlong(), ctypes.c_longlong(), ctypes.c_longlong(), ctypes.c_longlong()
        lib().mk_kv_sizes(self.h, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), ctypes.byref(d))
        return a.value, b.value, c.value, d.value

    def digest(self, seq=0):
        n = _check(lib().mk_kv_state_digest(self.h, seq, None, 0))
        out = (ctypes.c_ulonglong * n)()
        _check(lib().mk_kv_state_digest(self.h, seq, out, n))
        return list(out)

    def read_rows(self, seq, layer, w, g, p0, n, ring=False):
        """(values bytes [n][row_bytes], scales uint16 [n][8]) of logical rows p0 .. p0+n-1 (numpy arrays)."""
        import numpy as np
        bits = 8 if ring else (self.vbits if w else self.kbits)[layer]
        rb = 32 * bits
        vals = np.zeros((n, rb), np.uint8)
        sc = np.zeros((n, 8), np.uint16)
        _check(lib().mk_kv_read_rows(self.h, seq, layer, w, g, p0, n, 1 if ring else 0, vals.ctypes.data_as(ctypes.c_void_p),
                                     sc.ctypes.data_as(_P_u16)))
        return vals, sc

    def write_rows(self, seq, layer, w, g, p0, vals, scales, ring=False):
        """Write rows (values bytes [n][row_bytes], scales uint16 [n][8]) to logical positions p0 .. p0+n-1."""
        import numpy as np
        vals = np.ascontiguousarray(vals, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        _check(lib().mk_kv_write_rows(self.h, seq, layer, w, g, p0, vals.shape[0], 1 if ring else 0,
                                      vals.ctypes.data_as(ctypes.c_void_p), scales.ctypes.data_as(_P_u16)))

    def ring_snapshot(self, seq):
        """The window rings of sequence seq as a uint8 numpy array (header + rows)."""
        import numpy as np
        need = lib().mk_kv_ring_snapshot(self.h, seq, None, 0)
        if need < 0:
            raise KVError(last_error())
        buf = np.zeros(need, np.uint8)
        got = lib().mk_kv_ring_snapshot(self.h, seq, buf.ctypes.data_as(ctypes.c_void_p), need)
        if got != need:
            raise KVError(last_error())
        return buf

    def ring_restore(self, seq, pos, snap):
        import numpy as np
        snap = np.ascontiguousarray(snap, np.uint8)
        _check(lib().mk_kv_ring_restore(self.h, seq, pos, snap.ctypes.data_as(ctypes.c_void_p), snap.size))

    def profile(self, enable):
        """Start (1) / stop (0) kernel timing; returns {calls, attn_ms, combine_ms, append_ms} so far."""
        out = (ctypes.c_double * 4)()
        _check(lib().mk_kv_profile(self.h, int(enable), out, 4))
        return dict(zip(("calls", "attn_ms", "combine_ms", "append_ms"), list(out)))

    def config(self, key, value):
        """Knobs that never change results: "max_blocks" (attention grid cap, 0 = none), "occupancy" (decode
        workgroups per CU for one-token calls on small packed formats: 0 = by launch size, 2 or 3) and "wide" (T >= 5:
        1 = one pass of 8-wave workgroups, 0 = two 24-row passes)."""
        _check(lib().mk_kv_config(self.h, key.encode(), value))
