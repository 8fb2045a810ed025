"""Writes tests/golden/q5.npz: quantize / dequantize vectors produced by the REFERENCE's own formats/q5.cpp
(compiled from /root/reference by oracle/Makefile's `ref` target into oracle/_ref/, in the build container only) on
the same seeded inputs as formats.npz. The fixture is data: float inputs and the reference's outputs.

Run: python tests/golden/make_golden_q5.py   (needs oracle/_ref/libref_formats.so)
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", ".."))
sys.path.insert(0, os.path.dirname(__file__))
import oracle  # noqa: E402
from make_golden import cases  # noqa: E402


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_formats.so is not built (make -C oracle ref)")
    out = {}
    for name, w in cases():
        N, K = w.shape
        for G in (32, 64, 128):
            q = np.zeros(N * (K // 2 + K // 8), np.uint8)
            s = np.zeros(N * (K // G), np.uint16)
            m = np.zeros_like(s)
            assert ref.ref_quantize_q5(w.ctypes.data, N, K, G, q.ctypes.data, s.ctypes.data, m.ctypes.data) == 0
            d = np.zeros((N, K), np.float32)
            assert ref.ref_dequantize_q5(q.ctypes.data, s.ctypes.data, m.ctypes.data, N, K, G, d.ctypes.data) == 0
            tag = f"{name}_q5_g{G}"
            out[tag + "_w"] = w
            out[tag + "_q"], out[tag + "_s"], out[tag + "_m"], out[tag + "_deq"] = q, s, m, d
    # K % 128 != 0 is refused (the kernels' 16-byte aligned rows and planes)
    q = np.zeros(80, np.uint8); s = np.zeros(2, np.uint16); m = np.zeros(2, np.uint16)
    out["refuses_k64"] = np.array(ref.ref_quantize_q5(np.ones(64, np.float32).ctypes.data, 1, 64, 32, q.ctypes.data,
                                                      s.ctypes.data, m.ctypes.data) != 0)
    path = os.path.join(os.path.dirname(__file__), "q5.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes,", len(out), "arrays")


if __name__ == "__main__":
    main()
