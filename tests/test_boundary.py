"""The C-ABI boundary without a GPU: the library loads, exports every symbol include/strixite_moe.h declares, and
host-detectable preconditions fail with the reference's error behaviour (a StrixError naming the check) before any
device work."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    from strixite_amd import _lib

    L = _lib.lib()
    declared = _lib.declared_symbols()
    assert len(declared) >= 25
    missing = [n for n in declared if not hasattr(L, n)]
    assert not missing, missing
    assert L.strix_moe_abi_version() == 1


def test_cpp_header_declares_reference_signatures():
    hpp = open(os.path.join(ROOT, "include", "strixite_moe.hpp")).read()
    for name in ["moe_router", "check_router_error", "report_router_error", "moe_shared_add", "moe_shared_add_inject",
                 "moe_route_workspace_bytes", "moe_group_routes", "linear_q4_experts_gather_grouped",
                 "linear_q4_experts_gather_grouped_swiglu", "linear_q4_experts_combine_grouped",
                 "linear_q4_experts_gather", "linear_q4_experts_gather_swiglu", "linear_q4_experts_combine",
                 "check_expert_error", "report_expert_error", "swiglu", "linear_q8", "linear_bf16w"]:
        assert re.search(r"\b" + name + r"\(", hpp), name


def test_route_workspace_bytes_and_limits():
    from strixite_amd import moe

    n = moe.moe_route_workspace_bytes(16, 10, 512)
    S = 160
    # the reference's prefix (header 4 + offsets E+2 + slots S) comes first
    assert n >= (4 + 514 + S) * 4
    with pytest.raises(moe.StrixError, match="E = 1024"):
        moe.moe_route_workspace_bytes(1, 1, 1024)
    with pytest.raises(moe.StrixError):
        moe.moe_route_workspace_bytes(1 << 20, 2, 8)


def test_preconditions_raise_before_launch():
    """Null pointers, bad shapes and overlapping buffers are refused on the host (no device memory is touched)."""
    from strixite_amd import _lib

    L = _lib.lib()
    err = (C.c_uint32 * 3)()
    rc = L.strix_moe_router(None, 512, 1, 512, 10, None, 1, 0, None, None, 0, C.addressof(err), None)
    assert rc == 1 and b"null pointer" in L.strix_moe_last_error()
    buf = (C.c_uint8 * 4096)()
    p = C.addressof(buf)
    rc = L.strix_moe_router(p, 512, 1, 512, 33, None, 1, 0, p + 64, p + 128, 0, p + 256, None)
    assert rc == 1 and b"k = 33" in L.strix_moe_last_error()
    rc = L.strix_moe_router(p, 100, 1, 512, 8, None, 1, 0, p + 64, p + 128, 0, p + 256, None)
    assert rc == 1 and b"ld" in L.strix_moe_last_error()
    rc = L.strix_moe_router(p, 512, 1, 512, 8, None, 1, 0, p + 64, p + 64, 0, p + 256, None)
    assert rc == 1 and b"same buffer" in L.strix_moe_last_error()
    # overlapping output / input of the router projection
    rc = L.strix_linear_bf16w(p, p, p + 8, 1, 4, 64, 1, 0, None)
    assert rc == 1 and b"overlaps" in L.strix_moe_last_error()
    # a Q4 group size the K step does not divide
    v = _lib.QView(p, p, p, 64, 256, 64)
    rc = L.strix_linear_q4_experts_gather_grouped_swiglu(p, C.byref(v), 2, p, 1 << 20, 4, 2, p + 2048, 1, 2, None, 0)
    assert rc == 1 and b"group size" in L.strix_moe_last_error()
    # too small a workspace
    v = _lib.QView(p, p, p, 64, 256, 128)
    rc = L.strix_linear_q4_experts_gather_grouped_swiglu(p, C.byref(v), 2, p, 16, 4, 2, p + 2048, 1, 2, None, 0)
    assert rc == 1 and b"workspace" in L.strix_moe_last_error()
    rc = L.strix_moe_shared_add_inject(p, p + 1024, p + 2048, 1, 1, 16, 0, p + 8, p + 3000, 4, 1, p + 3500, None)
    assert rc == 1 and b"overlaps" in L.strix_moe_last_error()


def test_host_error_words_report_like_the_reference():
    from strixite_amd import _lib

    L = _lib.lib()
    ok = (C.c_uint32 * 3)(0, 0, 0)
    assert L.strix_report_router_error(C.addressof(ok), b"L0") == 0
    bad = (C.c_uint32 * 3)(1, 7, 512)
    assert L.strix_report_router_error(C.addressof(bad), b"L3 moe") == 1
    msg = L.strix_moe_last_error()
    assert b"L3 moe" in msg and b"token 7" in msg and b"expert 512" in msg
    bad = (C.c_uint32 * 3)(1, 0xFFFFFFFF, 42)
    assert L.strix_report_expert_error(C.addressof(bad), b"experts") == 1
    assert b"expert id -1 at slot 42" in L.strix_moe_last_error()
