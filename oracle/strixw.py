"""strixw parsed in numpy -- TEST INFRASTRUCTURE ONLY: the checker for the library's C++ reader and HBM loader.

An independent restatement of the file layout the reference writes and reads (strixite formats/strixw.cpp:251-336
writer, :338-466 reader): header, index records, component placement, the hash (``orc_strixw_hash64`` in
moe_oracle.c). Pinned by the fixture under tests/golden/ that the reference's own writer produced. It reads a whole
file into memory: for the small files the tests use.
"""
from __future__ import annotations

import struct

import numpy as np

from . import lib

MAGIC = b"STRIXWT\0"
ENCODINGS = {1: "q4", 2: "q4-chunk-major", 3: "bf16", 4: "f32", 5: "i64", 6: "q8", 7: "q8-chunk-major", 8: "q6",
             9: "q5"}
ROLES = {0: "data", 1: "q", 2: "scale", 3: "min"}


def hash64(b: bytes | np.ndarray) -> int:
    a = np.frombuffer(bytes(b), np.uint8) if not isinstance(b, np.ndarray) else np.ascontiguousarray(b).view(np.uint8)
    return int(lib().orc_strixw_hash64(a.ctypes.data if a.size else None, a.size))


def component_sizes(enc: int, shape: list[int], G: int) -> list[tuple[str, int]]:
    """(role, bytes) in file order (strixite formats/strixw.cpp:143-200)."""
    if enc in (3, 4, 5):
        n = int(np.prod(shape))
        return [("data", n * {3: 2, 4: 4, 5: 8}[enc])]
    N, K = shape
    code = {1: N * K // 2, 2: N * K // 2, 6: N * K, 7: N * K, 8: N * (K // 2 + K // 4), 9: N * (K // 2 + K // 8)}[enc]
    return [("q", code), ("scale", N * (K // G) * 2), ("min", N * (K // G) * 2)]


class File:
    """Header, metadata and tensor records of one strixw file; ``data(name, role)`` the component's bytes."""

    def __init__(self, path: str):
        with open(path, "rb") as f:
            self.buf = f.read()
        b = self.buf
        if len(b) < 128 or b[:8] != MAGIC:
            raise ValueError("not a strixw file")
        (self.version, hsize, ioff, ibytes, self.data_offset, fbytes, ihash) = struct.unpack_from("<IIQQQQQ", b, 8)
        if struct.unpack_from("<Q", b, 120)[0] != hash64(b[:120]):
            raise ValueError("header hash")
        if hsize != 128 or ioff != 128 or fbytes != len(b) or ioff + ibytes > len(b):
            raise ValueError("header fields")
        idx = b[ioff:ioff + ibytes]
        if ihash != hash64(idx):
            raise ValueError("index hash")
        at = 0

        def take(fmt):
            nonlocal at
            v = struct.unpack_from("<" + fmt, idx, at)
            at += struct.calcsize("<" + fmt)
            return v if len(v) > 1 else v[0]

        def text(n):
            nonlocal at
            v = idx[at:at + n].decode()
            at += n
            return v

        self.meta = {}
        for _ in range(take("I")):
            k = text(take("H"))
            self.meta[k] = text(take("I"))
        self.tensors = []
        for _ in range(take("I")):
            t = {"name": text(take("H")), "encoding": take("B")}
            nd = take("B")
            t["shape"] = [take("q") for _ in range(nd)]
            t["group_size"], t["experts"] = take("q"), take("q")
            t["parts"] = []
            for _ in range(take("H")):
                src = text(take("H"))
                t["parts"].append((src, take("q"), take("q")))
            t["components"] = []
            for _ in range(take("B")):
                role, off, nb, h = take("BQQQ")
                t["components"].append((ROLES[role], off, nb, h))
            want = component_sizes(t["encoding"], t["shape"], t["group_size"])
            if [(r, n) for r, _, n, _ in t["components"]] != want:
                raise ValueError(f"components of {t['name']}")
            self.tensors.append(t)
        if at != len(idx):
            raise ValueError("index trailing bytes")
        self.by_name = {t["name"]: t for t in self.tensors}

    def data(self, name: str, role: str) -> np.ndarray:
        for r, off, nb, _ in self.by_name[name]["components"]:
            if r == role:
                return np.frombuffer(self.buf, np.uint8, nb, off)
        raise KeyError((name, role))

    def verify(self) -> None:
        for t in self.tensors:
            for r, off, nb, h in t["components"]:
                if hash64(self.buf[off:off + nb]) != h:
                    raise ValueError(f"hash of {t['name']} {r}")

    def qspec(self, name: str):
        """(bits, q, scale, minv, G) numpy arrays of a q4 / q8 row-major tensor, the oracle's weight form."""
        t = self.by_name[name]
        bits = {1: 4, 6: 8}[t["encoding"]]
        return (bits, self.data(name, "q").copy(), self.data(name, "scale").view(np.uint16).copy(),
                self.data(name, "min").view(np.uint16).copy(), t["group_size"])

    def moe_layer(self, prefix: str, k: int) -> dict:
        """The oracle's layer weights (oracle.moe_layer's ``w``) for one decoder layer's MoE sublayer
        (strixite runtime/qwen4exp.cpp:147-156)."""
        m = prefix + "mlp."
        r = self.by_name[m + "router"]
        E = r["shape"][0] - 1
        I = self.by_name[m + "experts_down"]["shape"][1]
        w = {"E": E, "k": k, "I": I,
             "router": self.data(m + "router", "data").view(np.uint16).reshape(r["shape"]).copy(),
             "gu": self.qspec(m + "experts_gate_up"), "dn": self.qspec(m + "experts_down")}
        if m + "shared_expert.gate_up" in self.by_name:
            w["sh_gu"] = self.qspec(m + "shared_expert.gate_up")
            w["sh_dn"] = self.qspec(m + "shared_expert.down_proj.weight")
        else:
            w["shared_stacked"] = True
        return w
