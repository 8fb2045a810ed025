"""CPU oracle for the quantized MoE FFN path -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``liboracle_moe.so`` (plain C, ``moe_oracle.c``), the CPU restatement of the reference
algorithm (strixite ``kernels/moe_router.hip``, ``kernels/moe_grouped.hip``, ``kernels/linear_q4.hip``,
``kernels/swiglu.hip``, ``formats/q4.cpp``, ``formats/q8.cpp``; each C function cites its lines). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this package, and only as the checker
or the timed CPU baseline. The product path (``strixite_amd``) never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.environ.get("ORACLE_LIB") or os.path.join(_HERE, "liboracle_moe.so")  # ORACLE_LIB: the sanitizer build
_REF = os.path.join(_HERE, "_ref", "libref_formats.so")

_i64, _u64, _u32, _f32, _i32 = C.c_int64, C.c_uint64, C.c_uint32, C.c_float, C.c_int32
_p = C.c_void_p

TENSOR = {  # tensor ids of the seeded generator (shared with strixite_amd/csrc/synth.hip)
    "x": 1, "router": 2, "gu_q": 3, "gu_s": 4, "dn_q": 5, "dn_s": 6,
    "sh_gu_q": 7, "sh_gu_s": 8, "sh_dn_q": 9, "sh_dn_s": 10, "logits": 11, "zipf": 12,
}


def build(force: bool = False) -> None:
    """Compiles liboracle_moe.so (and, where /root/reference exists, oracle/_ref) with the Makefile here."""
    if force or not os.path.exists(_LIB):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []) + ["all"], check=True)
    if os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = C.CDLL(_LIB)
        L.orc_f32_to_bf16.restype = C.c_uint16
        L.orc_strixw_hash64.restype = _u64
        L.orc_strixw_hash64.argtypes = [_p, _u64]
        L.orc_f32_to_bf16.argtypes = [_f32]
        L.orc_bf16_to_f32.restype = _f32
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_splitmix64.restype = _u64
        L.orc_splitmix64.argtypes = [_u64]
        L.orc_tensor_key.restype = _u64
        L.orc_tensor_key.argtypes = [_u64, _u32, _u32]
        L.orc_gen_normal.restype = _f32
        L.orc_gen_normal.argtypes = [_u64, _u64, _f32]
        L.orc_gen_bf16_normal.argtypes = [_u64, _f32, _p, _i64]
        L.orc_gen_q4.argtypes = [_u64, _u64, _i64, _i64, _i64, _p, _p, _p]
        L.orc_gen_q8.argtypes = [_u64, _u64, _i64, _i64, _i64, _p, _p, _p]
        L.orc_gen_uniform_pm1.argtypes = [_u64, _p, _i64]
        L.orc_quantize_q4.restype = C.c_int
        L.orc_quantize_q4.argtypes = [_p, _i64, _i64, _i64, _p, _p, _p]
        L.orc_quantize_q8.restype = C.c_int
        L.orc_quantize_q8.argtypes = [_p, _i64, _i64, _i64, _p, _p, _p]
        L.orc_dequantize.argtypes = [C.c_int, _p, _p, _p, _i64, _i64, _i64, _p]
        L.orc_router_logits.argtypes = [_p, _p, _i64, _i64, _i64, _p, _i64, _p, C.c_int]
        L.orc_canonical_dot.restype = _f32
        L.orc_canonical_dot.argtypes = [_p, _p, _i64]
        L.orc_topk.restype = C.c_int
        L.orc_topk.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _i64, _i32, _p, _p, _p]
        L.orc_group_routes.argtypes = [_p, _i64, _i64, _i64, _p, _p, _p]
        L.orc_experts_gate_up_swiglu.argtypes = [_p, _p, _i64, _p, _i64, _i64, _p, C.c_int]
        L.orc_experts_down.argtypes = [_p, _p, _i64, _p, _i64, _i64, _p, C.c_int]
        L.orc_dense.argtypes = [_p, _p, _i64, _p, C.c_int]
        L.orc_swiglu_bf16.argtypes = [_p, _p, _i64, _i64]
        L.orc_combine.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _p]
        L.orc_moe_layer.restype = C.c_int
        L.orc_moe_layer.argtypes = [_p, _p, C.c_int]
        _lib = L
    return _lib


def ref_lib():
    """The reference's own formats/q4.cpp + q8.cpp + q5.cpp (oracle/_ref), or None where it is not built."""
    if not os.path.exists(_REF):
        return None
    L = C.CDLL(_REF)
    for n in ("ref_quantize_q4", "ref_quantize_q8", "ref_quantize_q5"):
        getattr(L, n).restype = C.c_int
        getattr(L, n).argtypes = [_p, _i64, _i64, _i64, _p, _p, _p]
    for n in ("ref_dequantize_q4", "ref_dequantize_q8", "ref_dequantize_q5"):
        getattr(L, n).restype = C.c_int
        getattr(L, n).argtypes = [_p, _p, _p, _i64, _i64, _i64, _p]
    return L


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def default_threads() -> int:
    return max(1, min(os.cpu_count() or 1, 16))


# ---- bf16 ----------------------------------------------------------------------------------------------------
def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """RNE, NaN kept quiet (strixite common/bf16.hpp:19-26), vectorized with the same integer arithmetic."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nonfin = (u & 0x7F800000) == 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nf = ((u >> 16) | np.where((u & 0x007FFFFF) != 0, 0x40, 0)).astype(np.uint16)
    return np.where(nonfin, nf, r).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- generator -----------------------------------------------------------------------------------------------
def tensor_key(seed: int, tensor: str | int, layer: int = 0) -> int:
    t = TENSOR[tensor] if isinstance(tensor, str) else tensor
    return int(lib().orc_tensor_key(seed, t, layer))


def gen_bf16_normal(key: int, sigma: float, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().orc_gen_bf16_normal(key, sigma, _ptr(out), out.size)
    return out


def gen_q(bits: int, key_codes: int, key_scales: int, rows: int, K: int, G: int):
    q = np.empty(rows * K // (2 if bits == 4 else 1), dtype=np.uint8)
    s = np.empty(rows * (K // G), dtype=np.uint16)
    m = np.empty_like(s)
    fn = lib().orc_gen_q4 if bits == 4 else lib().orc_gen_q8
    fn(key_codes, key_scales, rows, K, G, _ptr(q), _ptr(s), _ptr(m))
    return q, s, m


def gen_uniform_pm1(key: int, shape) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    lib().orc_gen_uniform_pm1(key, _ptr(out), out.size)
    return out


# ---- formats -------------------------------------------------------------------------------------------------
def quantize(bits: int, w: np.ndarray, G: int):
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    q = np.zeros(N * K // (2 if bits == 4 else 1), dtype=np.uint8)
    s = np.zeros(N * (K // G), dtype=np.uint16)
    m = np.zeros_like(s)
    fn = lib().orc_quantize_q4 if bits == 4 else lib().orc_quantize_q8
    if fn(_ptr(w), N, K, G, _ptr(q), _ptr(s), _ptr(m)) != 0:
        raise ValueError("quantize: bad shape, group size or non-finite weight")
    return q, s, m


def dequantize(bits: int, q, s, m, N: int, K: int, G: int) -> np.ndarray:
    w = np.empty((N, K), dtype=np.float32)
    lib().orc_dequantize(bits, _ptr(q), _ptr(s), _ptr(m), N, K, G, _ptr(w))
    return w


# ---- router / routing ----------------------------------------------------------------------------------------
def router_logits(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None, threads: int | None = None):
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib().orc_router_logits(_ptr(x), _ptr(w), M, N, K, _ptr(bias), 0 if bias is None else bias.size, _ptr(y),
                            threads or default_threads())
    return y


def topk(logits: np.ndarray, E: int, k: int, shared: np.ndarray | None = None, shared_ld: int = 1,
         shared_id: int = 0):
    M, ld = logits.shape
    A = k + (1 if shared is not None else 0)
    ids = np.empty((M, A), dtype=np.int32)
    coef = np.empty((M, A), dtype=np.float32)
    err = np.zeros(3, dtype=np.uint32)
    rc = lib().orc_topk(_ptr(logits), ld, M, E, k, _ptr(shared), shared_ld, shared_id, _ptr(ids), _ptr(coef),
                        _ptr(err))
    if rc != 0:
        raise ValueError("topk: bad arguments")
    return ids, coef, err


def group_routes(ids: np.ndarray, E: int):
    M, A = ids.shape
    offsets = np.empty(E + 2, dtype=np.int32)
    slots = np.empty(M * A, dtype=np.int32)
    err = np.zeros(3, dtype=np.uint32)
    lib().orc_group_routes(_ptr(np.ascontiguousarray(ids)), M, A, E, _ptr(offsets), _ptr(slots), _ptr(err))
    return offsets, slots, err


# ---- expert math ---------------------------------------------------------------------------------------------
class QView(C.Structure):
    _fields_ = [("bits", C.c_int), ("q", _p), ("scale", _p), ("minv", _p), ("N", _i64), ("K", _i64), ("G", _i64)]


def qview(bits, q, s, m, N, K, G) -> QView:
    return QView(bits, _ptr(q), _ptr(s), _ptr(m), N, K, G)


def experts_gate_up_swiglu(x, view: QView, E, ids, threads=None):
    M, A = ids.shape
    I = view.N // E // 2
    h = np.empty((M * A, I), dtype=np.uint16)
    lib().orc_experts_gate_up_swiglu(_ptr(x), C.byref(view), E, _ptr(ids), M, A, _ptr(h),
                                     threads or default_threads())
    return h


def experts_down(h, view: QView, E, ids, threads=None):
    M, A = ids.shape
    N = view.N // E
    p = np.empty((M * A, N), dtype=np.float32)
    lib().orc_experts_down(_ptr(h), C.byref(view), E, _ptr(ids), M, A, _ptr(p), threads or default_threads())
    return p


# ---- the reference's F16 matrix-unit math (MoeMath::WmmaF16 kinds, Q4 experts) -----------------------------------
# strixite kernels/moe_grouped.hpp:32-33 and moe_grouped.hip:348-351: x rounded to F16 toward zero, each weight one
# F16 rounding of code * s + m with s and m rounded to F16, products summed in FP32 over all of K. numpy only: the
# sums here run in float64 (the GPU's FP32 order differs; tests allow for that).
def bf16_to_f16_rtz(b: np.ndarray) -> np.ndarray:
    """BF16 bits -> F16 rounded toward zero (strixite kernels/moe_grouped.hip:30-32, v_cvt_pkrtz of the value)."""
    v = bf16_to_f32(np.asarray(b, dtype=np.uint16))
    with np.errstate(over="ignore"):
        h = v.astype(np.float16)  # round to nearest even ...
    up = np.abs(h.astype(np.float32)) > np.abs(v)  # ... stepped back one F16 ulp where it rounded away from zero
    h[up] = np.nextafter(h[up], np.float16(0))
    return h


def q4_codes(q: np.ndarray, N: int, K: int) -> np.ndarray:
    """[N, K] Q4 codes: code 2j in the low nibble of byte j of a row, 2j + 1 in the high (formats/q4.cpp)."""
    b = np.asarray(q, dtype=np.uint8).reshape(N, K // 2)
    c = np.empty((N, K), dtype=np.uint8)
    c[:, 0::2], c[:, 1::2] = b & 0x0F, b >> 4
    return c


def q4_weights_f16(q, s, m, N: int, K: int, G: int) -> np.ndarray:
    """[N, K] F16 weights f16(code * f16(s) + f16(m)), one rounding (strixite kernels/wmma_gemm.hpp:116-141).
    code * s + m is exact in float64 (5 x 11 significant bits, exponents within F16's range), so numpy's correctly
    rounded float64 -> float16 conversion is the F16 FMA's result."""
    s16 = bf16_to_f32(np.asarray(s, dtype=np.uint16)).astype(np.float16).astype(np.float64).reshape(N, K // G, 1)
    m16 = bf16_to_f32(np.asarray(m, dtype=np.uint16)).astype(np.float16).astype(np.float64).reshape(N, K // G, 1)
    w = q4_codes(q, N, K).astype(np.float64).reshape(N, K // G, G) * s16 + m16
    return w.astype(np.float16).reshape(N, K)


def _f16_grouped(x_rows, w16, E, ids, row_of_slot):
    """FP32 outputs [M * A, N] of slot s = x16[row_of_slot(s)] . W16[ids[s]]^T (float64 sums rounded once)."""
    N = w16.shape[0] // E
    x16 = bf16_to_f16_rtz(x_rows).astype(np.float64)
    flat = np.asarray(ids).ravel()
    out = np.full((flat.size, N), np.nan, dtype=np.float32)
    for e in np.unique(flat):
        sl = np.nonzero(flat == e)[0]
        if 0 <= e < E:
            out[sl] = (x16[row_of_slot(sl)] @ w16[e * N:(e + 1) * N].astype(np.float64).T).astype(np.float32)
    return out


def experts_gate_up_swiglu_f16math(x, bits, q, s, m, N_total, K, G, E, ids):
    """h [M * A, I] (BF16 bits) = bf16(silu(g) * u) of the F16 math (strixite kernels/moe_grouped.hip:354, 348-351)."""
    assert bits == 4, "F16 matrix-unit math: Q4 experts"
    A = ids.shape[1]
    gu = _f16_grouped(x, q4_weights_f16(q, s, m, N_total, K, G), E, ids, lambda sl: sl // A)
    I = gu.shape[1] // 2
    g, u = gu[:, :I], gu[:, I:]
    with np.errstate(over="ignore", invalid="ignore"):
        return f32_to_bf16((g / (np.float32(1) + np.exp(-g))) * u)


def experts_gather_f16math(x, bits, q, s, m, N_total, K, G, E, ids):
    """FP32 per-slot gate_up (no SwiGLU) outputs [M * A, N] of the F16 math (x rows by slot // A; strixite
    kernels/moe_grouped.hip:348-351, the plain gather under an F16 kind)."""
    assert bits == 4, "F16 matrix-unit math: Q4 experts"
    A = ids.shape[1]
    return _f16_grouped(x, q4_weights_f16(q, s, m, N_total, K, G), E, ids, lambda sl: sl // A)


def experts_down_f16math(h, bits, q, s, m, N_total, K, G, E, ids):
    """FP32 per-slot down outputs [M * A, N] of the F16 math (h BF16 bits, slot rows)."""
    assert bits == 4, "F16 matrix-unit math: Q4 experts"
    return _f16_grouped(h, q4_weights_f16(q, s, m, N_total, K, G), E, ids, lambda sl: sl)


def dense(x, view: QView, threads=None):
    M = x.shape[0]
    y = np.empty((M, view.N), dtype=np.float32)
    lib().orc_dense(_ptr(x), C.byref(view), M, _ptr(y), threads or default_threads())
    return y


def swiglu_bf16(gu: np.ndarray, I: int) -> np.ndarray:
    rows = gu.shape[0]
    h = np.empty((rows, I), dtype=np.uint16)
    lib().orc_swiglu_bf16(_ptr(np.ascontiguousarray(gu)), _ptr(h), rows, I)
    return h


def combine(partial, ids, coef, E, N, s=None, gate_logit=None, gate_ld=1, resid=None):
    M, A = ids.shape
    y = np.empty((M, N), dtype=np.uint16)
    out = np.empty((M, N), dtype=np.uint16) if resid is not None else None
    lib().orc_combine(_ptr(partial), _ptr(ids), _ptr(coef), M, A, E, N, _ptr(s), _ptr(gate_logit), gate_ld,
                      _ptr(y), _ptr(resid), _ptr(out))
    return y, out


# ---- the sublayer --------------------------------------------------------------------------------------------
class _Layer(C.Structure):
    _fields_ = [("M", _i64), ("H", _i64), ("E", _i64), ("k", _i64), ("I", _i64), ("x", _p), ("router", _p),
                ("router_bias", _p), ("logits_in", _p), ("ld_in", _i64), ("gate_up", QView), ("down", QView),
                ("has_shared", C.c_int), ("sh_gate_up", QView), ("sh_down", QView), ("shared_stacked", C.c_int)]


class _LayerOut(C.Structure):
    _fields_ = [("logits", _p), ("ids", _p), ("coef", _p), ("offsets", _p), ("slots", _p), ("h", _p),
                ("partial", _p), ("sh_h", _p), ("sh_s", _p), ("y", _p), ("out", _p),
                ("err_router", _u32 * 3), ("err_route", _u32 * 3)]


def moe_layer(w: dict, x: np.ndarray, logits_in: np.ndarray | None = None, threads: int | None = None) -> dict:
    """The whole MoE sublayer on the CPU. ``w`` holds numpy arrays: router [E(+1), H] bf16 bits, router_bias
    (optional), gu/dn = (bits, q, s, m, G) for the stacked routed experts, sh_gu/sh_dn likewise (optional);
    shared_stacked: the shared expert is expert E of gu/dn, routed as slot k (ids / coef then [M, k + 1])."""
    M, H = x.shape
    E, k, I = w["E"], w["k"], w["I"]
    has_sh = "sh_gu" in w
    stacked = bool(w.get("shared_stacked")) and not has_sh
    ld = E + (1 if has_sh or stacked else 0)
    A = k + (1 if stacked else 0)
    Es = E + (1 if stacked else 0)
    keep = []

    def qv(spec, N, K):
        bits, q, s, m, G = spec
        keep.append((q, s, m))
        return qview(bits, q, s, m, N, K, G)

    L = _Layer()
    L.M, L.H, L.E, L.k, L.I = M, H, E, k, I
    L.x = _ptr(x)
    L.router = _ptr(w.get("router"))
    L.router_bias = _ptr(w.get("router_bias"))
    L.logits_in = _ptr(logits_in)
    L.ld_in = 0 if logits_in is None else logits_in.shape[1]
    L.gate_up = qv(w["gu"], Es * 2 * I, H)
    L.down = qv(w["dn"], Es * H, I)
    L.has_shared = 1 if has_sh else 0
    L.shared_stacked = 1 if stacked else 0
    if has_sh:
        L.sh_gate_up = qv(w["sh_gu"], 2 * I, H)
        L.sh_down = qv(w["sh_dn"], H, I)
    o = {
        "logits": np.empty((M, ld), np.float32), "ids": np.empty((M, A), np.int32),
        "coef": np.empty((M, A), np.float32), "offsets": np.empty(Es + 2, np.int32),
        "slots": np.empty(M * A, np.int32), "h": np.empty((M * A, I), np.uint16),
        "partial": np.empty((M * A, H), np.float32), "sh_h": np.empty((M, I), np.uint16),
        "sh_s": np.empty((M, H), np.uint16), "y": np.empty((M, H), np.uint16), "out": np.empty((M, H), np.uint16),
    }
    O = _LayerOut()
    for name in ("logits", "ids", "coef", "offsets", "slots", "h", "partial", "sh_h", "sh_s", "y", "out"):
        setattr(O, name, _ptr(o[name]))
    rc = lib().orc_moe_layer(C.byref(L), C.byref(O), threads or default_threads())
    if rc != 0:
        raise ValueError("moe_layer: bad arguments")
    o["err_router"] = np.array(list(O.err_router), dtype=np.uint32)
    o["err_route"] = np.array(list(O.err_route), dtype=np.uint32)
    return o
