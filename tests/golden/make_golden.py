"""Writes tests/golden/formats.npz: quantize / dequantize vectors produced by the REFERENCE's own
formats/q4.cpp and formats/q8.cpp (compiled from /root/reference by oracle/Makefile's `ref` target into
oracle/_ref/, in the build container only). The fixture is data: seeded float inputs and the reference's outputs.

Run: python tests/golden/make_golden.py   (needs oracle/_ref/libref_formats.so)
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", ".."))
import oracle  # noqa: E402


def cases():
    rng = np.random.default_rng(1234)
    N, K = 4, 256
    yield "normal", rng.standard_normal((N, K)).astype(np.float32) * 0.05
    w = rng.standard_normal((N, K)).astype(np.float32)
    w[1, :128] = 0.25  # constant groups: s = 0, codes 0
    w[2, :] = np.tile(np.array([0.0, 1.0], np.float32), K // 2)  # two-level groups
    yield "edge", w
    # values on quantization-grid midpoints: exercises round-half-to-even in the code rounding
    base = np.linspace(-1.0, 1.0, 16, dtype=np.float32)
    g = np.tile(np.concatenate([base, (base[:-1] + base[1:]) / 2, base[:1]]), K // 32 + 1)[:K]
    yield "halfway", np.stack([g, g * 3.0, g * 1e-3, -g]).astype(np.float32)
    yield "wide", (rng.standard_normal((N, K)) * np.logspace(-3, 3, K)).astype(np.float32)


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_formats.so is not built (make -C oracle ref)")
    out = {}
    for name, w in cases():
        N, K = w.shape
        for bits in (4, 8):
            for G in (32, 64, 128):
                q = np.zeros(N * K // (2 if bits == 4 else 1), np.uint8)
                s = np.zeros(N * (K // G), np.uint16)
                m = np.zeros_like(s)
                fq = ref.ref_quantize_q4 if bits == 4 else ref.ref_quantize_q8
                assert fq(w.ctypes.data, N, K, G, q.ctypes.data, s.ctypes.data, m.ctypes.data) == 0
                d = np.zeros((N, K), np.float32)
                fd = ref.ref_dequantize_q4 if bits == 4 else ref.ref_dequantize_q8
                assert fd(q.ctypes.data, s.ctypes.data, m.ctypes.data, N, K, G, d.ctypes.data) == 0
                tag = f"{name}_q{bits}_g{G}"
                out[tag + "_w"] = w
                out[tag + "_q"], out[tag + "_s"], out[tag + "_m"], out[tag + "_deq"] = q, s, m, d
        # the reference refuses non-finite input and bad group sizes: record its verdicts
    bad = np.array([[1.0, np.nan] * 16], np.float32)
    q = np.zeros(16, np.uint8); s = np.zeros(1, np.uint16); m = np.zeros(1, np.uint16)
    out["refuses_nan"] = np.array(ref.ref_quantize_q4(bad.ctypes.data, 1, 32, 32, q.ctypes.data, s.ctypes.data,
                                                      m.ctypes.data) != 0)
    out["refuses_g16"] = np.array(ref.ref_quantize_q4(np.ones(32, np.float32).ctypes.data, 1, 32, 16, q.ctypes.data,
                                                      s.ctypes.data, m.ctypes.data) != 0)
    path = os.path.join(os.path.dirname(__file__), "formats.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes,", len(out), "arrays")


if __name__ == "__main__":
    main()
