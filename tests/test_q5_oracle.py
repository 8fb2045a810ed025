"""The Q5 oracle (oracle/q5.py) against the golden vectors written by the reference's own quantize_q5 /
dequantize_q5 (tests/golden/q5.npz): codes, scales, mins and dequantized values bit for bit, plus the layout's
known positions."""
import os

import numpy as np

from oracle import q5

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "q5.npz"))


def test_quantize_and_dequantize_match_reference():
    tags = sorted({k[:-2] for k in GOLD.files if k.endswith("_w")})
    assert len(tags) == 12
    for t in tags:
        w = GOLD[t + "_w"]
        N, K = w.shape
        G = int(t.split("_g")[-1])
        q, s, m = q5.quantize(w, G)
        assert np.array_equal(q, GOLD[t + "_q"]), t
        assert np.array_equal(s, GOLD[t + "_s"]) and np.array_equal(m, GOLD[t + "_m"]), t
        d = q5.dequantize(GOLD[t + "_q"], GOLD[t + "_s"], GOLD[t + "_m"], N, K, G)
        assert np.array_equal(d.view(np.uint32), GOLD[t + "_deq"].view(np.uint32)), t
    assert bool(GOLD["refuses_k64"])


def test_layout_positions():
    K = 128
    c = np.zeros((1, K), np.uint8)
    c[0, 3], c[0, 8], c[0, 127] = 31, 16, 5
    b = q5.pack(c)
    assert b[1] == 0xF0 and b[64 + 0] == 0b1000 and b[64 + 1] == 0b1 and b[63] == 0x50
    assert np.array_equal(q5.codes(b, 1, K), c)
