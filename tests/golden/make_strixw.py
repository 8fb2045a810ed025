"""Writes tests/golden/layers.strixw and tests/golden/strixw.npz with the REFERENCE's own strixw writer and hash
(strixite formats/strixw.cpp, compiled from /root/reference by oracle/Makefile's `ref` target into oracle/_ref/, in
the build container only). The fixture is data: a two-layer MoE file in the converter's naming (layer 0: the shared
expert stacked as expert E, Q4 G128; layer 1: Q8 G64 routed experts and a separate Q8 shared expert), a few tensors
of the other encodings, hash vectors, and the reference reader's verdicts on corrupted copies.

Run: python tests/golden/make_strixw.py   (needs oracle/_ref/libref_strixw.so)
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))
import oracle  # noqa: E402
import oracle.strixw  # noqa: E402

REF = os.path.join(HERE, "..", "..", "oracle", "_ref", "libref_strixw.so")
LM = "model.language_model.layers."
ENC = {"q4": 1, "q4-chunk-major": 2, "bf16": 3, "f32": 4, "i64": 5, "q8": 6, "q6": 8, "q5": 9}


def key(layer, t):
    return oracle.tensor_key(7 + layer, t)


def qtensor(bits, layer, kq, ks, N, K, G):
    q, s, m = oracle.gen_q(bits, key(layer, kq), key(layer, ks), N, K, G)
    return [q, s, m]


def plan():
    """(name, encoding, shape, G, experts, parts [(source, rows)], components [arrays in file order])."""
    out = []
    rng = np.random.default_rng(5)
    # layer 0: H 128, E 4 (+ the stacked shared expert), I 128, Q4 G128
    H, E, I, P = 128, 4, 128, LM + "0.mlp."
    out.append((P + "router", "bf16", [E + 1, H], 0, 0, [(P + "gate.weight", E), (P + "shared_expert_gate.weight", 1)],
                [oracle.gen_bf16_normal(key(0, "router"), 0.02, ((E + 1) * H,))]))
    out.append((P + "experts_gate_up", "q4", [(E + 1) * 2 * I, H], 128, E + 1,
                [(P + "experts.gate_up_proj", E * 2 * I), (P + "shared_expert.gate_proj.weight", I),
                 (P + "shared_expert.up_proj.weight", I)],
                qtensor(4, 0, "gu_q", "gu_s", (E + 1) * 2 * I, H, 128)))
    out.append((P + "experts_down", "q4", [(E + 1) * H, I], 128, E + 1,
                [(P + "experts.down_proj", E * H), (P + "shared_expert.down_proj.weight", H)],
                qtensor(4, 0, "dn_q", "dn_s", (E + 1) * H, I, 128)))
    # layer 1: H 128, E 4, I 64, Q8 G64 routed; the shared expert separate, Q8 G64
    H, E, I, P = 128, 4, 64, LM + "1.mlp."
    out.append((P + "router", "bf16", [E + 1, H], 0, 0, [], [oracle.gen_bf16_normal(key(1, "router"), 0.02,
                                                                                    ((E + 1) * H,))]))
    out.append((P + "experts_gate_up", "q8", [E * 2 * I, H], 64, E, [], qtensor(8, 1, "gu_q", "gu_s", E * 2 * I, H, 64)))
    out.append((P + "experts_down", "q8", [E * H, I], 64, E, [], qtensor(8, 1, "dn_q", "dn_s", E * H, I, 64)))
    out.append((P + "shared_expert.gate_up", "q8", [2 * I, H], 64, 0, [],
                qtensor(8, 1, "sh_gu_q", "sh_gu_s", 2 * I, H, 64)))
    out.append((P + "shared_expert.down_proj.weight", "q8", [H, I], 64, 0, [],
                qtensor(8, 1, "sh_dn_q", "sh_dn_s", H, I, 64)))
    # the other encodings, listing only
    out.append(("model.language_model.norm.weight", "f32", [H], 0, 0, [], [rng.standard_normal(H).astype(np.float32)]))
    out.append(("extra.positions", "i64", [3], 0, 0, [], [np.array([1, -2, 1 << 40], np.int64)]))
    for name, enc, shape, G, code in (("extra.q4cm", "q4-chunk-major", [16, 64], 32, 16 * 32),
                                      ("extra.q6", "q6", [2, 64], 64, 2 * 48), ("extra.q5", "q5", [2, 128], 128, 2 * 80)):
        ng = shape[0] * (shape[1] // G)
        out.append((name, enc, shape, G, 0, [], [rng.integers(0, 256, code, dtype=np.uint8),
                                                 rng.integers(0, 65536, ng, dtype=np.uint16),
                                                 rng.integers(0, 65536, ng, dtype=np.uint16)]))
    return out


META = {"arch": "qwen4exp", "layout": "exp_gu=q4g128 (layer 0), q8g64 (layer 1)", "shared_expert": "mixed",
        "layers": "0,1", "note": "test fixture"}


def write_ref(ref, path, meta, tensors):
    nt = len(tensors)
    strs = lambda xs: (C.c_char_p * len(xs))(*[x.encode() for x in xs])  # noqa: E731
    shape = np.zeros((nt, 8), np.int64)
    for i, t in enumerate(tensors):
        shape[i, :len(t[2])] = t[2]
    parts = [p for t in tensors for p in t[5]]
    arrays = [np.ascontiguousarray(a) for t in tensors for a in t[6]]
    data = (C.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])
    rc = ref.ref_strixw_write(path.encode(), len(meta), strs(list(meta)), strs(list(meta.values())), nt,
                              strs([t[0] for t in tensors]), (C.c_int * nt)(*[ENC[t[1]] for t in tensors]),
                              (C.c_int * nt)(*[len(t[2]) for t in tensors]), shape.ctypes.data,
                              (C.c_int64 * nt)(*[t[3] for t in tensors]), (C.c_int64 * nt)(*[t[4] for t in tensors]),
                              (C.c_int * nt)(*[len(t[5]) for t in tensors]), strs([p[0] for p in parts]),
                              (C.c_int64 * max(1, len(parts)))(*[p[1] for p in parts]), data)
    assert rc == 0, ref.ref_strixw_error()


def corruptions(buf: bytes):
    """(name, bytes) variants of a valid file; the reference reader's verdict on each is recorded."""
    b = bytearray(buf)
    yield "header_flip", bytes(b[:60]) + bytes([b[60] ^ 1]) + bytes(b[61:])
    yield "index_flip", bytes(b[:200]) + bytes([b[200] ^ 0x10]) + bytes(b[201:])
    yield "truncated", bytes(b[:-1])
    yield "appended", bytes(b) + b"\0"
    dflip = bytearray(b)
    dflip[-1] ^= 0xFF  # inside the last component (the file ends with it)
    yield "data_flip", bytes(dflip)
    pflip = bytearray(b)
    pflip[-5] ^= 0xFF  # alignment padding between the last two components: not hashed
    yield "padding_flip", bytes(pflip)
    for v in (0, 1, 5):  # a version outside / inside the readable range, header hash recomputed
        x = bytearray(b)
        x[8:12] = np.uint32(v).tobytes()
        x[120:128] = np.uint64(oracle.strixw.hash64(bytes(x[:120]))).tobytes()
        yield f"version_{v}", bytes(x)


def main():
    if not os.path.exists(REF):
        raise SystemExit("oracle/_ref/libref_strixw.so is not built (make -C oracle ref)")
    ref = C.CDLL(REF)
    ref.ref_strix_hash64.restype = C.c_uint64
    ref.ref_strix_hash64.argtypes = [C.c_void_p, C.c_size_t]
    ref.ref_strix_hash64_pieces.restype = C.c_uint64
    ref.ref_strix_hash64_pieces.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_int]
    ref.ref_strixw_error.restype = C.c_char_p
    ref.ref_strixw_check.argtypes = [C.c_char_p, C.c_int]
    ref.ref_strixw_write.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p]
    path = os.path.join(HERE, "layers.strixw")
    write_ref(ref, path, META, plan())
    assert ref.ref_strixw_check(path.encode(), 1) == 0, ref.ref_strixw_error()

    out = {}
    rng = np.random.default_rng(11)
    blob = rng.integers(0, 256, 4200, dtype=np.uint8)
    lengths = np.array(list(range(0, 72)) + [95, 96, 97, 127, 128, 129, 1000, 4099, 4200], np.int64)
    out["hash_blob"], out["hash_lengths"] = blob, lengths
    out["hash_values"] = np.array([ref.ref_strix_hash64(blob.ctypes.data, int(n)) for n in lengths], np.uint64)
    cuts = [[1], [31, 32, 33], [7, 8, 64, 65, 999], [0, 0, 500], [32 * i for i in range(1, 31)]]
    out["piece_cuts"] = np.array([c + [-1] * (32 - len(c)) for c in cuts], np.int64)
    out["piece_values"] = np.array([ref.ref_strix_hash64_pieces(blob.ctypes.data, 1000,
                                                                (C.c_size_t * len(c))(*c), len(c)) for c in cuts],
                                   np.uint64)
    buf = open(path, "rb").read()
    names, opened, verified = [], [], []
    tmp = path + ".tmp"
    for name, b in corruptions(buf):
        with open(tmp, "wb") as f:
            f.write(b)
        names.append(name)
        opened.append(ref.ref_strixw_check(tmp.encode(), 0) == 0)
        verified.append(ref.ref_strixw_check(tmp.encode(), 1) == 0)
    os.remove(tmp)
    out["corrupt_names"] = np.array(names)
    out["corrupt_open_ok"], out["corrupt_verify_ok"] = np.array(opened), np.array(verified)
    np.savez_compressed(os.path.join(HERE, "strixw.npz"), **out)
    print(path, len(buf), "bytes;", dict(zip(names, zip(opened, verified))))


if __name__ == "__main__":
    main()
