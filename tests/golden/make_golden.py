"""Write tests/golden/kv_golden.npz: seeded inputs and the oracle's outputs for the KV path (test fixture).

    python tests/golden/make_golden.py

The reference holds no golden vectors for this path, so these vectors are produced by the oracle (oracle/kv_oracle.c),
itself pinned by closed forms and invariants (tests/test_oracle_*.py).  They freeze the exact bytes the oracle produced
when it was pinned, for regression checks of the oracle and for GPU checks that need no CPU arithmetic at run time.
Inputs are stored as fp16 (exactly representable), so the fixture stays small.

Contents:
  rows_x          [64][256] fp16  row inputs: N(0,1) with outlier channels, plus crafted blocks (zero block, one
                                  nonzero, +-ties, tiny and huge magnitudes)
  rows_<b><r>_q   main-store bytes of every row for bits b in 4..8, r = 'r' (rotated) or 'n'
  rows_<b><r>_s   their fp16 scales (uint16)
  rows_<r>_rq/rs  the window-ring q8 bytes / scales (the same for every b)
  fwht_x, fwht_y  [8][256] fp32: inputs and the FWHT outputs
  attn_*          one layer with preset F's packed sides (K 5-bit rotated, V 6-bit), no window, L = 40 positions
                  (one full tile and a ragged one): K, V inputs [40][4][256] fp16, Q [1][24][256] fp32, and the fp64
                  attention on the stored operands as fp32 [1][24][256]
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import oracle  # noqa: E402
from kvcase import expected_attention  # noqa: E402

HD = 256


def row_inputs(rng):
    x = rng.standard_normal((64, HD)).astype(np.float32)
    x[:, rng.choice(HD, 4, replace=False)] *= 12.0
    x[1, :32] = 0.0                          # an all-zero block
    x[2, :32] = 0.0
    x[2, 5] = -3.0                           # a block with one nonzero value
    x[3, 32:64] = np.tile([1.5, -1.5], 16)   # |x| ties: the larger x wins
    x[4] *= 1e-3                             # small magnitudes
    x[5] *= 200.0                            # large magnitudes (fp16-safe after the 1/127 and 1/h scales)
    return x.astype(np.float16)


def main():
    rng = np.random.default_rng(20260101)
    out = {}
    x = row_inputs(rng)
    out["rows_x"] = x
    xf = x.astype(np.float32)
    for r, rot in (("n", 0), ("r", 1)):
        for b in (4, 5, 6, 7, 8):
            mq, ms, rq, rs = oracle.store_rows(xf, rot, b, ring=True)
            out[f"rows_{b}{r}_q"] = mq
            out[f"rows_{b}{r}_s"] = ms
        out[f"rows_{r}_rq"] = rq
        out[f"rows_{r}_rs"] = rs
    fx = rng.standard_normal((8, HD)).astype(np.float32)
    out["fwht_x"] = fx
    out["fwht_y"] = np.stack([oracle.fwht(v) for v in fx])
    L, win = 40, 0
    K = rng.standard_normal((L, 4, HD)).astype(np.float16)
    V = rng.standard_normal((L, 4, HD)).astype(np.float16)
    Q = rng.standard_normal((1, 24, HD)).astype(np.float32)
    ws = oracle.ws(L, win)
    out.update(attn_K=K, attn_V=V, attn_Q=Q, attn_L=np.int32(L), attn_win=np.int32(win), attn_ws=np.int32(ws),
               attn_y=expected_attention(oracle, Q, K.astype(np.float32), V.astype(np.float32), 1, True, False, 5, 6, ws,
                                         win > 0, win > 0))
    path = os.path.join(HERE, "kv_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
