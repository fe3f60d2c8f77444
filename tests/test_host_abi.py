"""The C-ABI library without a GPU: it loads, exports every symbol include/qwen38_kv.h declares, and its host-only
logic (MK_KV grammar, window geometry, T capping, error reporting) agrees with the oracle and the reference's rules."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_names():
    txt = open(os.path.join(ROOT, "include", "qwen38_kv.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(mk_\w+)\s*\(", txt)))


def test_exports_every_declared_symbol(qkv):
    lib = ctypes.CDLL(qkv.LIB_PATH)
    names = header_names()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(qkv.SIGNATURES), "binding table and header disagree"


def test_geometry_matches_oracle(qkv, oracle):
    for win in (0, 512, 1024, 2048, 4096):
        assert qkv.ring_rows(win) == oracle.kvrc(win)
        for L in list(range(1, 7000, 13)) + [101600, 262144]:
            assert qkv.window_start(L, win) == oracle.ws(L, win)
    for n in range(0, 3000, 11):
        for T in range(1, 9):
            assert qkv.cap_T(n, T) == oracle.cap_T(n, T)


def test_parse_spec(qkv):
    kb, vb, kr, vr = qkv.parse_spec("K*=5r,V*=6", 16)
    assert kb == [5] * 16 and vb == [6] * 16 and kr == [1] * 16 and vr == [0] * 16
    kb, vb, kr, vr = qkv.parse_spec("", 4)
    assert kb == vb == [8] * 4 and kr == vr == [0] * 4
    kb, vb, kr, vr = qkv.parse_spec("*=4,K2=7r,V=6r", 4)   # later items override; empty slot = all
    assert kb == [4, 4, 7, 4] and vb == [6] * 4 and kr == [0, 0, 1, 0] and vr == [1] * 4
    kb, vb, kr, vr = qkv.parse_spec(",,V1=7,,K+1=4r,", 3)   # empty items skipped; the slot is strtol syntax
    assert kb == [8, 4, 8] and vb == [8, 7, 8] and kr == [0, 1, 0] and vr == [0] * 3
    for bad, msg in [("K1=5=6", "expected 4..8"), ("K1=", "expected 4..8"), ("Kx=5", "bad slot"), ("K-1=5", "bad slot"),
                     ("K3=5", "bad slot")]:
        with pytest.raises(qkv.KVError, match=msg):
            qkv.parse_spec(bad, 3)
    for bad, msg in [("X=5", "bad item"), ("K=9", "expected 4..8"), ("K99=5", "bad slot"), ("K*=5x", "expected"),
                     ("K1", "bad item"), ("=5", "bad item")]:
        with pytest.raises(qkv.KVError, match=msg):
            qkv.parse_spec(bad, 16)


def test_new_rejects_bad_arguments(qkv):
    for args in [("", 0, 0, 0, 1, 100, 0, 0), ("", 0, 0, 18, 1, 100, 0, 0), ("", 0, 0, 1, 0, 100, 0, 0),
                 ("", 0, 0, 1, 1, 100, 48, 0), ("", -1, 0, 1, 1, 100, 0, 0), ("K=3", 0, 0, 1, 1, 100, 0, 0)]:
        spec = args[0].encode() if args[0] else None
        assert not qkv.lib().mk_kv_new(spec, *args[1:])
        assert qkv.last_error()


def test_null_handle_errors(qkv):
    assert qkv.lib().mk_kv_rewind(None, 0, 0) == -1
    assert "null" in qkv.last_error()
    qkv.lib().mk_free(None)


def test_no_gpu_new_fails_cleanly(qkv):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(qkv.KVError):
        qkv.KVStore("K*=5r,V*=6", 2048, n_layers=1, ctx=1024)
