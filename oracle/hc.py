"""CPU oracle for the hyper-connection mix (strixite kernels/hc.hpp) -- TEST INFRASTRUCTURE ONLY.

float64 closed forms of hc_mix_down and hc_mix_up (strixite kernels/hc.hpp:3-18 for the semantics, :31-50 for the
interfaces; the per-32-code chunk form s * sum(x * code) + m * sum(x) of kernels/hc.hip:104-113 is the same sum in
exact arithmetic) and the chunk-major weight layout (strixite formats/q4.hpp:43-55, formats/q4.cpp:101-119). Only
``tests/`` import this module. ``brute_*`` restate the same formulas as scalar loops for tiny inputs: the pins of the
vectorized forms.
"""
from __future__ import annotations

import numpy as np

from . import bf16_to_f32, q4_codes

STREAMS = 4


def weights64(bits: int, q, s, m, N: int, K: int, G: int) -> np.ndarray:
    """[N, K] float64 w = code * scale + min of a row-major Q4 / Q8 weight (formats/q4.hpp:3-6, q8.hpp:3-10),
    exact (no FP32 rounding)."""
    codes = q4_codes(q, N, K) if bits == 4 else np.asarray(q, np.uint8).reshape(N, K)
    sc = bf16_to_f32(np.asarray(s).view(np.uint16)).reshape(N, K // G).astype(np.float64)
    mn = bf16_to_f32(np.asarray(m).view(np.uint16)).reshape(N, K // G).astype(np.float64)
    return codes.astype(np.float64) * np.repeat(sc, G, axis=1) + np.repeat(mn, G, axis=1)


def to_chunk_major(bits: int, q, s, m, N: int, K: int, G: int):
    """Row-major Q4 / Q8 arrays -> chunk-major (strixite formats/q4.cpp:101-119): chunk c of row n's 16 (Q4) or 32
    (Q8) code bytes at [(c N + n) * bytes], group g's scale / min at [g N + n]."""
    cb = 16 if bits == 4 else 32
    qc = np.asarray(q, np.uint8).reshape(N, K // 32, cb).transpose(1, 0, 2).reshape(-1)
    sc = np.asarray(s).reshape(N, K // G).T.reshape(-1)
    mc = np.asarray(m).reshape(N, K // G).T.reshape(-1)
    return np.ascontiguousarray(qc), np.ascontiguousarray(sc), np.ascontiguousarray(mc)


def hc_mix_down(x: np.ndarray, w64: np.ndarray, d: int, r: int, inject: bool, eps: float):
    """x [T, 4 d] -> (h [T, r], w_in [T, 4] or None, inv [T, 4]): inv = 1/sqrt(mean(X_s^2) + eps), a = sum_s inv_s
    (W_s . X_s), h = silu(a / 4), w_in = 2 sigmoid(a / 4) for the 4 rows after r (strixite kernels/hc.hpp:31-36)."""
    T = x.shape[0]
    X = np.asarray(x, np.float64).reshape(T, STREAMS, d)
    inv = 1.0 / np.sqrt((X * X).mean(axis=2) + eps)
    R = w64.shape[0]
    part = np.einsum("tsj,nsj->tns", X, w64.reshape(R, STREAMS, d))
    z = (part * inv[:, None, :]).sum(axis=2) / STREAMS
    h = z[:, :r] / (1.0 + np.exp(-z[:, :r]))
    w_in = 2.0 / (1.0 + np.exp(-z[:, r:r + STREAMS])) if inject else None
    return h, w_in, inv


def hc_mix_up(h: np.ndarray, wup64: np.ndarray, x: np.ndarray, norm_w: np.ndarray, inv: np.ndarray, d: int):
    """u [T, d] = (1/4) sum_s sigmoid(W_up[s d + j] . h[t]) * X[t, s d + j] inv[t, s] (1 + norm_w[s d + j]), W_up
    [4 d, r] (strixite kernels/hc.hpp:38-50)."""
    T = x.shape[0]
    with np.errstate(over="ignore"):  # exp overflow to inf gives the gate's limit 0 exactly
        g = 1.0 / (1.0 + np.exp(-(np.asarray(h, np.float64) @ wup64.T)))
    n = np.asarray(x, np.float64).reshape(T, STREAMS, d) * np.asarray(inv, np.float64)[:, :, None] * (
        1.0 + np.asarray(norm_w, np.float64).reshape(STREAMS, d))
    return (g.reshape(T, STREAMS, d) * n).sum(axis=1) / STREAMS


def brute_mix_down(x, w64, d, r, inject, eps):
    """hc_mix_down as scalar loops (tiny inputs)."""
    import math

    T, R = x.shape[0], w64.shape[0]
    h = [[0.0] * r for _ in range(T)]
    w_in = [[0.0] * STREAMS for _ in range(T)]
    inv = [[0.0] * STREAMS for _ in range(T)]
    for t in range(T):
        for s in range(STREAMS):
            inv[t][s] = 1.0 / math.sqrt(sum(float(x[t, s * d + j]) ** 2 for j in range(d)) / d + eps)
        for n in range(R):
            a = 0.0
            for s in range(STREAMS):
                a += inv[t][s] * sum(float(w64[n, s * d + j]) * float(x[t, s * d + j]) for j in range(d))
            z = a / STREAMS
            if n < r:
                h[t][n] = z / (1.0 + math.exp(-z))
            elif inject:
                w_in[t][n - r] = 2.0 / (1.0 + math.exp(-z))
    return np.array(h), (np.array(w_in) if inject else None), np.array(inv)


def brute_mix_up(h, wup64, x, norm_w, inv, d):
    """hc_mix_up as scalar loops (tiny inputs)."""
    import math

    T, r = h.shape
    u = np.zeros((T, d))
    for t in range(T):
        for j in range(d):
            acc = 0.0
            for s in range(STREAMS):
                row = s * d + j
                a = sum(float(wup64[row, i]) * float(h[t, i]) for i in range(r))
                acc += (1.0 / (1.0 + math.exp(-a))) * float(x[t, row]) * float(inv[t, s]) * (1.0 + float(norm_w[row]))
            u[t, j] = acc / STREAMS
    return u
