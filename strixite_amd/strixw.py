"""strixw files from Python over the library's C++ reader, writer and HBM loader (include/strixite_strixw.hpp,
C-ABI strix_strixw_* in include/strixite_moe.h). The classes mirror strixite formats/strixw.hpp (StrixwFile,
StrixwWriter) and runtime/strixw_loader.hpp (StrixwDevice); a failed check raises StrixError with the library's
message."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L

ENCODING = {"q4": 1, "q4-chunk-major": 2, "bf16": 3, "f32": 4, "i64": 5, "q8": 6, "q8-chunk-major": 7, "q6": 8,
            "q5": 9}
ENCODING_NAME = {v: k for k, v in ENCODING.items()}
ROLE = {"data": 0, "q": 1, "scale": 2, "min": 3}
ROLE_NAME = {v: k for k, v in ROLE.items()}


def hash64(data) -> int:
    """The format's 64-bit hash (strixite formats/strixw.hpp:58 strix_hash64)."""
    a = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if isinstance(data, (bytes, bytearray)) else data)
    return int(L.lib().strix_strixw_hash64(a.ctypes.data if a.nbytes else None, a.nbytes))


@dataclass
class Tensor:
    name: str
    encoding: str
    shape: list
    group_size: int
    experts: int
    parts: list = field(default_factory=list)       # [(source, row_offset, rows)]
    components: list = field(default_factory=list)  # [(role, offset, bytes, hash)]


class StrixwFile:
    """A strixw file mapped and validated by the library's reader."""

    def __init__(self, path: str):
        self.path = path
        h = C.c_void_p()
        L.check(L.lib().strix_strixw_open(path.encode(), C.byref(h)))
        self._h = h
        fb, do, ver, nt, nm = C.c_uint64(), C.c_uint64(), C.c_uint32(), C.c_int64(), C.c_int64()
        L.check(L.lib().strix_strixw_info(h, C.byref(fb), C.byref(do), C.byref(ver), C.byref(nt), C.byref(nm)))
        self.file_bytes, self.data_offset, self.version = fb.value, do.value, ver.value
        self.meta = {}
        for i in range(nm.value):
            k, v = C.c_char_p(), C.c_char_p()
            L.check(L.lib().strix_strixw_meta(h, i, C.byref(k), C.byref(v)))
            self.meta[k.value.decode()] = v.value.decode()
        self.tensors = []
        for i in range(nt.value):
            info = L.StrixwTensorInfo()
            L.check(L.lib().strix_strixw_tensor(h, i, C.byref(info)))
            t = Tensor(info.name.decode(), ENCODING_NAME.get(info.encoding, str(info.encoding)),
                       list(info.shape[:info.ndim]), info.group_size, info.experts)
            for j in range(info.nparts):
                src, off, rows = C.c_char_p(), C.c_int64(), C.c_int64()
                L.check(L.lib().strix_strixw_part(h, i, j, C.byref(src), C.byref(off), C.byref(rows)))
                t.parts.append((src.value.decode(), off.value, rows.value))
            t.components = [(ROLE_NAME[info.role[c]], info.offset[c], info.bytes[c], info.hash[c])
                            for c in range(info.ncomponents)]
            self.tensors.append(t)
        self.by_name = {t.name: t for t in self.tensors}

    def verify_hashes(self, threads: int = 4) -> None:
        L.check(L.lib().strix_strixw_verify(self._h, threads))

    def close(self) -> None:
        if self._h:
            L.lib().strix_strixw_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write(path: str, meta: dict, tensors: list) -> None:
    """StrixwWriter over the library: tensors = [{"name", "encoding", "shape", "group_size"=0, "experts"=0,
    "parts"=[(source, rows)], "data": {role: ndarray}}], written in index order."""
    n = len(tensors)
    plans = (L.StrixwPlan * n)()
    keep = []
    for i, t in enumerate(tensors):
        p = plans[i]
        p.name = t["name"].encode()
        p.encoding = ENCODING[t["encoding"]]
        p.ndim = len(t["shape"])
        for d, v in enumerate(t["shape"]):
            p.shape[d] = v
        p.group_size, p.experts = t.get("group_size", 0), t.get("experts", 0)
        parts = t.get("parts", [])
        p.nparts = len(parts)
        if parts:
            srcs = (C.c_char_p * len(parts))(*[s.encode() for s, _ in parts])
            rows = (C.c_int64 * len(parts))(*[r for _, r in parts])
            keep += [srcs, rows]
            p.part_sources, p.part_rows = srcs, rows
    keys = (C.c_char_p * max(1, len(meta)))(*[k.encode() for k in meta])
    vals = (C.c_char_p * max(1, len(meta)))(*[v.encode() for v in meta.values()])
    w = C.c_void_p()
    L.check(L.lib().strix_strixw_writer_create(path.encode(), len(meta), keys, vals, n, plans, C.byref(w)))
    try:
        for i, t in enumerate(tensors):
            for role, arr in t["data"].items():
                a = np.ascontiguousarray(arr)
                L.check(L.lib().strix_strixw_writer_write(w, i, ROLE[role], a.ctypes.data, a.nbytes))
        L.check(L.lib().strix_strixw_writer_finish(w))
    finally:
        L.lib().strix_strixw_writer_destroy(w)


class StrixwDevice:
    """The file's data region in one HBM allocation on the current device (strixite runtime/strixw_loader.hpp)."""

    def __init__(self, path: str, read_threads: int = 8):
        h = C.c_void_p()
        L.check(L.lib().strix_strixw_device_load(path.encode(), read_threads, C.byref(h)))
        self._h = h
        nb, sec = C.c_uint64(), C.c_double()
        L.check(L.lib().strix_strixw_device_info(h, C.byref(nb), C.byref(sec)))
        self.device_bytes, self.load_seconds = nb.value, sec.value

    def ptr(self, name: str, role: str = "data") -> int:
        p = C.c_void_p()
        L.check(L.lib().strix_strixw_device_ptr(self._h, name.encode(), ROLE[role], C.byref(p)))
        return p.value

    def moe_layer(self, prefix: str, top_k: int):
        """The MoE sublayer of one decoder layer (strixite runtime/qwen4exp.cpp:147-156) as a moe.MoeLayer whose
        views point into this allocation (the layer keeps this object alive)."""
        from .moe import MoeLayer

        w = L.LayerWeights()
        L.check(L.lib().strix_strixw_moe_layer(self._h, prefix.encode(), top_k, C.byref(w)))
        return MoeLayer.from_view(w, owner=self)

    def free(self) -> None:
        if self._h:
            L.lib().strix_strixw_device_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
