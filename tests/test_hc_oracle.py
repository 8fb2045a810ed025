"""Pins of the hyper-connection mix oracle (oracle/hc.py) on the CPU: the vectorized float64 forms against scalar
loops on tiny inputs, closed-form special cases, and the chunk-major layout's known positions (strixite
formats/q4.cpp:101-119)."""
import numpy as np

import oracle as orc
from oracle import hc


def _q(bits, N, K, G, seed):
    return orc.gen_q(bits, orc.tensor_key(seed, "gu_q"), orc.tensor_key(seed, "gu_s"), N, K, G)


def test_vectorized_matches_brute_force():
    d, r, T = 32, 6, 3
    rng = np.random.default_rng(0)
    x = rng.standard_normal((T, 4 * d))
    for bits, G in ((4, 32), (8, 64)):
        q, s, m = _q(bits, r + 4, 4 * d, G, 3)
        w = hc.weights64(bits, q, s, m, r + 4, 4 * d, G)
        h, wi, inv = hc.hc_mix_down(x, w, d, r, True, 1e-6)
        hb, wib, invb = hc.brute_mix_down(x, w, d, r, True, 1e-6)
        assert np.allclose(h, hb, rtol=1e-12, atol=1e-14)
        assert np.allclose(wi, wib, rtol=1e-12) and np.allclose(inv, invb, rtol=1e-12)
        qu, su, mu = _q(bits, 4 * d, 32, 32, 4)
        wu = hc.weights64(bits, qu, su, mu, 4 * d, 32, 32)
        hh = rng.standard_normal((T, 32)) * 0.1
        nw = rng.standard_normal(4 * d) * 0.1
        assert np.allclose(hc.hc_mix_up(hh, wu, x, nw, inv, d), hc.brute_mix_up(hh, wu, x, nw, inv, d), rtol=1e-11)


def test_closed_forms():
    d, r, T = 64, 5, 2
    x = np.full((T, 4 * d), 3.0)
    zero = np.zeros((r + 4, 4 * d))
    h, wi, inv = hc.hc_mix_down(x, zero, d, r, True, 0.5)
    assert np.all(h == 0) and np.allclose(wi, 1.0)  # silu(0) = 0, 2 sigmoid(0) = 1
    assert np.allclose(inv, 1.0 / np.sqrt(9.0 + 0.5))
    # zero up weights: every gate is sigmoid(0) = 1/2, so u = (1/4) sum_s X inv (1 + w) / 2
    nw = np.linspace(-0.5, 0.5, 4 * d)
    u = hc.hc_mix_up(np.ones((T, 32)), np.zeros((4 * d, 32)), x, nw, inv, d)
    ref = 0.5 * 3.0 * inv[:, :1] * (1 + nw.reshape(4, d)).sum(axis=0)[None, :] / 4  # inv alike over streams here
    assert np.allclose(u, ref)
    # one stream scaled: inv of that stream only changes (the RMS of each stream is its own)
    x2 = x.copy()
    x2[:, d:2 * d] *= 2
    _, _, inv2 = hc.hc_mix_down(x2, zero, d, r, False, 0.5)
    assert np.allclose(inv2[:, 0], inv[:, 0]) and np.allclose(inv2[:, 1], 1.0 / np.sqrt(36.0 + 0.5))


def test_weights64_matches_reference_dequantize():
    for bits, G in ((4, 64), (8, 32)):
        q, s, m = _q(bits, 5, 128, G, 7)
        w = hc.weights64(bits, q, s, m, 5, 128, G)
        assert np.allclose(w, orc.dequantize(bits, q, s, m, 5, 128, G), rtol=1e-6, atol=1e-7)


def test_chunk_major_positions():
    N, K, G = 3, 64, 32
    for bits, cb in ((4, 16), (8, 32)):
        q = np.arange(N * K * bits // 8, dtype=np.uint8)
        s = np.arange(N * K // G, dtype=np.uint16)
        qc, sc, _ = hc.to_chunk_major(bits, q, s, s, N, K, G)
        for n in range(N):
            for c in range(K // 32):
                assert np.array_equal(qc[(c * N + n) * cb:(c * N + n + 1) * cb],
                                      q.reshape(N, -1)[n, c * cb:(c + 1) * cb])
            for g in range(K // G):
                assert sc[g * N + n] == s.reshape(N, -1)[n, g]
