"""The oracle against the committed golden vectors (tests/golden/kv_golden.npz, written by make_golden.py): any change
of the oracle's bytes or attention output shows here."""
import os

import numpy as np
import pytest

from kvcase import expected_attention

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kv_golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(G, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("rot", ["n", "r"])
@pytest.mark.parametrize("bits", [4, 5, 6, 7, 8])
def test_rows_match_golden(oracle, gold, bits, rot):
    x = gold["rows_x"].astype(np.float32)
    mq, ms, rq, rs = oracle.store_rows(x, rot == "r", bits, ring=True)
    assert np.array_equal(mq, gold[f"rows_{bits}{rot}_q"])
    assert np.array_equal(ms, gold[f"rows_{bits}{rot}_s"])
    assert np.array_equal(rq, gold[f"rows_{rot}_rq"])
    assert np.array_equal(rs, gold[f"rows_{rot}_rs"])


def test_fwht_matches_golden(oracle, gold):
    y = np.stack([oracle.fwht(v) for v in gold["fwht_x"]])
    assert np.array_equal(y, gold["fwht_y"])


def test_attention_matches_golden(oracle, gold):
    L, ws, win = int(gold["attn_L"]), int(gold["attn_ws"]), int(gold["attn_win"])
    y = expected_attention(oracle, gold["attn_Q"], gold["attn_K"].astype(np.float32), gold["attn_V"].astype(np.float32),
                           1, True, False, 5, 6, ws, win > 0, win > 0)
    assert y.shape == gold["attn_y"].shape and L == gold["attn_K"].shape[0]
    assert np.array_equal(y, gold["attn_y"])
