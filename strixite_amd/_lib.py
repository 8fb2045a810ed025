"""ctypes binding of libstrixite_moe.so (include/strixite_moe.h). Loads the in-tree build only; there is no
fallback: without the library every call raises."""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("STRIX_MOE_LIB") or os.path.join(HERE, "libstrixite_moe.so")

_p, _i64, _i32, _u32, _u64, _f32, _int, _sz = (C.c_void_p, C.c_int64, C.c_int32, C.c_uint32, C.c_uint64, C.c_float,
                                               C.c_int, C.c_size_t)


class StrixError(RuntimeError):
    """A failed host-side precondition (strixite's strix::Error)."""


class GpuError(StrixError):
    """The HIP runtime reported an error."""


class QView(C.Structure):  # strix_qview
    _fields_ = [("q", _p), ("scale", _p), ("minv", _p), ("N", _i64), ("K", _i64), ("G", _i64)]


class SharedAdd(C.Structure):  # strix_moe_shared_add_t
    _fields_ = [("s", _p), ("gate_logit", _p), ("gate_ld", _i64), ("gate_index", _u32), ("err", _p)]


class InjectArgs(C.Structure):  # strix_moe_inject_t
    _fields_ = [("xs", _p), ("w_in", _p), ("streams", _i64)]


class LayerWeights(C.Structure):  # strix_moe_layer_weights
    _fields_ = [("H", _i64), ("E", _i64), ("k", _i64), ("I", _i64), ("router", _p), ("router_bias", _p),
                ("routed_bits", _int), ("gate_up", QView), ("down", QView), ("has_shared", _int),
                ("sh_gate_up", QView), ("sh_down", QView), ("shared_stacked", _int)]


class StrixwTensorInfo(C.Structure):  # strix_strixw_tensor_info
    _fields_ = [("name", C.c_char_p), ("encoding", _int), ("ndim", _int), ("shape", _i64 * 8), ("group_size", _i64),
                ("experts", _i64), ("nparts", _i64), ("ncomponents", _int), ("role", _int * 4),
                ("offset", _u64 * 4), ("bytes", _u64 * 4), ("hash", _u64 * 4)]


class StrixwPlan(C.Structure):  # strix_strixw_plan_t
    _fields_ = [("name", C.c_char_p), ("encoding", _int), ("ndim", _int), ("shape", _i64 * 8), ("group_size", _i64),
                ("experts", _i64), ("nparts", _i64), ("part_sources", C.POINTER(C.c_char_p)),
                ("part_rows", C.POINTER(_i64))]


_SIGS = {
    "strix_moe_abi_version": (_int, []),
    "strix_moe_last_error": (C.c_char_p, []),
    "strix_linear_bf16w": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _int, _p]),
    "strix_moe_router": (_int, [_p, _i64, _i64, _i64, _i64, _p, _i64, _i32, _p, _p, _int, _p, _p]),
    "strix_check_router_error": (_int, [_p, C.c_char_p]),
    "strix_report_router_error": (_int, [_p, C.c_char_p]),
    "strix_moe_shared_add": (_int, [_p, _p, _p, _i64, _i64, _i64, _u32, _int, _p, _p]),
    "strix_moe_shared_add_inject": (_int, [_p, _p, _p, _i64, _i64, _i64, _u32, _p, _p, _i64, _int, _p, _p]),
    "strix_moe_route_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "strix_moe_group_routes": (_int, [_p, _i64, _i64, _i64, _p, _sz, _p, _p]),
    "strix_linear_q4_experts_gather_grouped": (_int, [_p, C.POINTER(QView), _i64, _p, _sz, _i64, _i64, _p, _int,
                                                      _int, _p]),
    "strix_linear_q4_experts_gather_grouped_swiglu": (_int, [_p, C.POINTER(QView), _i64, _p, _sz, _i64, _i64, _p,
                                                             _int, _int, _p, _int]),
    "strix_linear_q4_experts_combine_grouped": (_int, [_p, C.POINTER(QView), _i64, _p, _p, _p, _sz, _p, _i64, _i64,
                                                       _p, _int, _int, _p, C.POINTER(SharedAdd), _int]),
    "strix_linear_q8_experts_gather_grouped_swiglu": (_int, [_p, C.POINTER(QView), _i64, _p, _sz, _i64, _i64, _p,
                                                             _int, _int, _p, _int]),
    "strix_linear_q8_experts_combine_grouped": (_int, [_p, C.POINTER(QView), _i64, _p, _p, _p, _sz, _p, _i64, _i64,
                                                       _p, _int, _int, _p, C.POINTER(SharedAdd), _int]),
    "strix_linear_q4_experts_gather": (_int, [_p, C.POINTER(QView), _i64, _p, _i64, _i64, _p, _int, _p, _p]),
    "strix_linear_q4_experts_gather_swiglu": (_int, [_p, C.POINTER(QView), _i64, _p, _i64, _i64, _p, _int, _p, _p]),
    "strix_linear_q4_experts_combine": (_int, [_p, C.POINTER(QView), _i64, _p, _p, _i64, _i64, _p, _int, _p, _p]),
    "strix_linear_q5_experts_gather_grouped": (_int, [_p, C.POINTER(QView), _i64, _p, _sz, _i64, _i64, _p, _int,
                                                      _int, _p]),
    "strix_linear_q5_experts_gather_grouped_swiglu": (_int, [_p, C.POINTER(QView), _i64, _p, _sz, _i64, _i64, _p,
                                                             _int, _int, _p, _int]),
    "strix_linear_q5_experts_combine_grouped": (_int, [_p, C.POINTER(QView), _i64, _p, _p, _p, _sz, _p, _i64, _i64,
                                                       _p, _int, _int, _p, C.POINTER(SharedAdd), _int]),
    "strix_linear_q5_experts_gather": (_int, [_p, C.POINTER(QView), _i64, _p, _i64, _i64, _p, _int, _p, _p]),
    "strix_linear_q5_experts_gather_swiglu": (_int, [_p, C.POINTER(QView), _i64, _p, _i64, _i64, _p, _int, _p, _p]),
    "strix_linear_q5_experts_combine": (_int, [_p, C.POINTER(QView), _i64, _p, _p, _i64, _i64, _p, _int, _p, _p]),
    "strix_check_expert_error": (_int, [_p, C.c_char_p]),
    "strix_report_expert_error": (_int, [_p, C.c_char_p]),
    "strix_swiglu": (_int, [_p, _p, _i64, _i64, _int, _p]),
    "strix_linear_q4": (_int, [_p, C.POINTER(QView), _p, _i64, _int, _int, _p]),
    "strix_linear_q8": (_int, [_p, C.POINTER(QView), _p, _i64, _int, _int, _p]),
    "strix_moe_layer_workspace_bytes": (_i64, [C.POINTER(LayerWeights), _i64]),
    "strix_moe_layer_context_create": (_int, [C.POINTER(_p)]),
    "strix_moe_layer_context_destroy": (_int, [_p]),
    "strix_calib_mfma_peak": (_i64, [_i64, _int, _p, _p]),
    "strix_calib_read_peak": (_int, [_p, _i64, _i64, _p, _p]),
    "strix_calib_bf16_round": (_int, [_p, _p, _i64, _p]),
    "strix_moe_layer_noalloc_max_bytes": (_i64, []),
    "strix_moe_layer_forward_noalloc": (_int, [C.POINTER(LayerWeights), _p, _i64, _p, _p, _p, _p, _p, _p, _p]),
    "strix_moe_layer_forward": (_int, [C.POINTER(LayerWeights), _p, _i64, _p, _p, _p, _p, _p, _p, _sz, _p, _p, _p,
                                       C.POINTER(InjectArgs)]),
    "strix_hc_inject": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _p]),
    "strix_hc_mix_down": (_int, [_p, _p, _int, _i64, _i64, _i64, _i64, _int, C.c_float, _p, _p, _p, _int, _p]),
    "strix_hc_mix_up": (_int, [_p, _p, _int, _p, _p, _p, _i64, _i64, _i64, _p, _int, _p]),
    "strix_strixw_hash64": (_u64, [_p, _sz]),
    "strix_strixw_open": (_int, [C.c_char_p, C.POINTER(_p)]),
    "strix_strixw_close": (_int, [_p]),
    "strix_strixw_info": (_int, [_p, C.POINTER(_u64), C.POINTER(_u64), C.POINTER(_u32), C.POINTER(_i64),
                                 C.POINTER(_i64)]),
    "strix_strixw_tensor": (_int, [_p, _i64, C.POINTER(StrixwTensorInfo)]),
    "strix_strixw_find": (_int, [_p, C.c_char_p, C.POINTER(_i64)]),
    "strix_strixw_part": (_int, [_p, _i64, _i64, C.POINTER(C.c_char_p), C.POINTER(_i64), C.POINTER(_i64)]),
    "strix_strixw_meta": (_int, [_p, _i64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p)]),
    "strix_strixw_verify": (_int, [_p, _int]),
    "strix_strixw_writer_create": (_int, [C.c_char_p, _i64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), _i64,
                                          C.POINTER(StrixwPlan), C.POINTER(_p)]),
    "strix_strixw_writer_write": (_int, [_p, _i64, _int, _p, _sz]),
    "strix_strixw_writer_finish": (_int, [_p]),
    "strix_strixw_writer_destroy": (_int, [_p]),
    "strix_strixw_device_load": (_int, [C.c_char_p, _int, C.POINTER(_p)]),
    "strix_strixw_device_free": (_int, [_p]),
    "strix_strixw_device_info": (_int, [_p, C.POINTER(_u64), C.POINTER(C.c_double)]),
    "strix_strixw_device_ptr": (_int, [_p, C.c_char_p, _int, C.POINTER(_p)]),
    "strix_strixw_moe_layer": (_int, [_p, C.c_char_p, _i64, C.POINTER(LayerWeights)]),
    "strix_synth_tensor_key": (_u64, [_u64, _u32, _u32]),
    "strix_synth_bf16_normal": (_int, [_u64, _f32, _p, _i64, _p]),
    "strix_synth_q_weight": (_int, [_int, _u64, _u64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "strix_synth_uniform_pm1": (_int, [_u64, _p, _i64, _p]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library (raises if it was never built: python strixite_amd/build.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise StrixError(f"{LIB_PATH} is missing: build it with `python strixite_amd/build.py` "
                             "(or __graft_entry__.build()); there is no fallback path")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def check(rc: int) -> None:
    """Turns a C-ABI return code into StrixError / GpuError with the library's message."""
    if rc == 0:
        return
    msg = lib().strix_moe_last_error().decode(errors="replace")
    raise (GpuError if rc == 2 else StrixError)(msg)


def declared_symbols() -> list[str]:
    """Every function include/strixite_moe.h declares."""
    import re

    hdr = os.path.join(os.path.dirname(HERE), "include", "strixite_moe.h")
    return sorted(set(re.findall(r"\b(strix_[a-z0-9_]+)\s*\(", open(hdr).read())))
