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


def _sigmoid(v):
    import math

    return 1.0 / (1.0 + math.exp(-v))


def test_down_closed_form_nonzero_weights():
    """Constant streams (stream s holds v_s everywhere) and per-(row, stream) constant weights c[n, s]: the dot of row
    n with stream s is d c[n, s] v_s, the inverse RMS is 1 / sqrt(v_s^2 + eps), so a_n = sum_s d c[n, s] v_s /
    sqrt(v_s^2 + eps) and z = a / 4 -- computed here element by element with the textbook silu and logistic. A form
    with z = a, an inverse RMS paired with the wrong stream, or a mean over 4 d instead of d fails it."""
    import math

    d, r, eps = 32, 3, 0.25
    v = [0.5, -1.5, 2.0, 3.0]
    c = np.array([[0.01 * (n + 1) * (s + 1) * (-1) ** s for s in range(4)] for n in range(r + 4)])
    x = np.concatenate([np.full(d, vs) for vs in v])[None, :].repeat(2, axis=0)
    w = np.repeat(c, d, axis=1)  # row n: c[n, 0] over stream 0's d columns, then c[n, 1], ...
    h, wi, inv = hc.hc_mix_down(x, w, d, r, True, eps)
    for n in range(r + 4):
        a = sum(d * c[n, s] * v[s] / math.sqrt(v[s] ** 2 + eps) for s in range(4))
        z = a / 4
        want = z * _sigmoid(z) if n < r else 2 * _sigmoid(z)
        got = h[0, n] if n < r else wi[0, n - r]
        assert abs(got - want) <= 1e-12 * max(1.0, abs(want)), (n, got, want)
    assert np.allclose(inv[0], [1 / math.sqrt(vs * vs + eps) for vs in v], rtol=1e-14)
    # the same numbers from the mutated forms differ by far more than rounding
    a0 = sum(d * c[0, s] * v[s] / math.sqrt(v[s] ** 2 + eps) for s in range(4))
    assert abs(a0 * _sigmoid(a0) - h[0, 0]) > 1e-3  # z = a instead of a / 4
    swapped = sum(d * c[0, s] * v[s] / math.sqrt(v[3 - s] ** 2 + eps) for s in range(4)) / 4
    assert abs(swapped * _sigmoid(swapped) - h[0, 0]) > 1e-3  # inverse RMS of another stream


def test_up_closed_form_one_hot_rows():
    """W_up [4 d, r] with one 1 per row: row s d + j picks column p(s, j) of h, so the gate of (t, s, j) is
    sigmoid(h[t, p(s, j)]) whatever the other columns hold. With constant streams v_s and norm weight w_s, u[t, j] =
    (1/4) sum_s sigmoid(h[t, p(s, j)]) v_s inv_s (1 + w_s), computed element by element. Reading W_up transposed
    (W_up[:, i] as row i) or dropping the 1/4 fails it."""
    import math

    d, r, T = 32, 40, 2
    v = [1.0, -2.0, 0.5, 4.0]
    inv = np.array([[0.5, 0.25, 2.0, 1.0], [1.0, 1.0, 1.0, 1.0]])
    nwv = [0.1, -0.2, 0.3, 0.0]
    x = np.concatenate([np.full(d, vs) for vs in v])[None, :].repeat(T, axis=0)
    nw = np.concatenate([np.full(d, w) for w in nwv])
    h = np.arange(T * r, dtype=np.float64).reshape(T, r) * 0.07 - 1.3
    pick = lambda s, j: (7 * s + 3 * j + 1) % r
    wu = np.zeros((4 * d, r))
    for s in range(4):
        for j in range(d):
            wu[s * d + j, pick(s, j)] = 1.0
    u = hc.hc_mix_up(h, wu, x, nw, inv, d)
    for t in range(T):
        for j in range(d):
            want = sum(_sigmoid(h[t, pick(s, j)]) * v[s] * inv[t, s] * (1 + nwv[s]) for s in range(4)) / 4
            assert abs(u[t, j] - want) <= 1e-12 * max(1.0, abs(want)), (t, j)
    # a transposed reading of the same bytes ([r, 4 d] row-major taken as W_up rows) gives other gates
    wt = wu.reshape(-1)[: 4 * d * r].reshape(r, 4 * d).T
    assert not np.allclose(hc.hc_mix_up(h, np.ascontiguousarray(wt), x, nw, inv, d), u, rtol=1e-6)
