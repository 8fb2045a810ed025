"""CPU oracle for the Q5 expert format (strixite formats/q5.hpp:3-13, :33-37) -- TEST INFRASTRUCTURE ONLY.

numpy restatement of the layout (per row a low plane [K/2] of 4-bit codes, low nibble = even k, then a high plane
[K/8] of bit 4, code k at bit k % 8 of byte k / 8), the quantizer (s = bf16((max - min) / 31), m = bf16(min), code =
clamp(rne((w - m) / s), 0, 31), FP32; s == 0: code 0) and the exact dequantization (code * s, then + m, two FP32
roundings). Pinned by tests/golden/q5.npz, written by the reference's own quantize_q5 / dequantize_q5. Only
``tests/`` import this module.
"""
from __future__ import annotations

import numpy as np

from . import bf16_to_f32, f32_to_bf16


def row_bytes(K: int) -> int:
    return K // 2 + K // 8


def codes(q, N: int, K: int) -> np.ndarray:
    """[N, K] 5-bit codes from the two planes."""
    b = np.asarray(q, np.uint8).reshape(N, row_bytes(K))
    lo = np.empty((N, K), np.uint8)
    lo[:, 0::2], lo[:, 1::2] = b[:, :K // 2] & 0x0F, b[:, :K // 2] >> 4
    hi = np.unpackbits(b[:, K // 2:], axis=1, bitorder="little")
    return lo | (hi << 4)


def pack(c: np.ndarray) -> np.ndarray:
    """[N, K] codes (0..31) -> the two-plane row bytes, flattened."""
    N, K = c.shape
    lo = (c[:, 0::2] & 0x0F) | ((c[:, 1::2] & 0x0F) << 4)
    hi = np.packbits((c >> 4) & 1, axis=1, bitorder="little")
    return np.concatenate([lo.astype(np.uint8), hi], axis=1).reshape(-1)


def quantize(w: np.ndarray, G: int):
    """w [N, K] FP32 -> (q bytes, scale bits, min bits), formats/q5.cpp's arithmetic."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    g = w.reshape(N, K // G, G)
    lo, hi = g.min(axis=2), g.max(axis=2)
    sb = f32_to_bf16(((hi - lo) / np.float32(31.0)).astype(np.float32))
    mb = f32_to_bf16(lo)
    s, m = bf16_to_f32(sb)[:, :, None], bf16_to_f32(mb)[:, :, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(((g - m) / s).astype(np.float32))
    c = np.where(s > 0, np.clip(r, 0, 31), 0).astype(np.uint8).reshape(N, K)
    return pack(c), sb.reshape(-1), mb.reshape(-1)


def dequantize(q, s, m, N: int, K: int, G: int) -> np.ndarray:
    """[N, K] FP32 code * s then + m (two roundings)."""
    sc = np.repeat(bf16_to_f32(np.asarray(s).view(np.uint16)).reshape(N, K // G), G, axis=1)
    mn = np.repeat(bf16_to_f32(np.asarray(m).view(np.uint16)).reshape(N, K // G), G, axis=1)
    return (codes(q, N, K).astype(np.float32) * sc).astype(np.float32) + mn


def weights64(q, s, m, N: int, K: int, G: int) -> np.ndarray:
    """[N, K] float64 code * s + m, exact."""
    sc = np.repeat(bf16_to_f32(np.asarray(s).view(np.uint16)).reshape(N, K // G).astype(np.float64), G, axis=1)
    mn = np.repeat(bf16_to_f32(np.asarray(m).view(np.uint16)).reshape(N, K // G).astype(np.float64), G, axis=1)
    return codes(q, N, K).astype(np.float64) * sc + mn
