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
    assert L.strix_moe_abi_version() == 4


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
    # a group size outside the format's 32 / 64 / 128
    v = _lib.QView(p, p, p, 64, 256, 16)
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


REF = "/root/reference"
REF_HEADERS = ["kernels/moe_router.hpp", "kernels/moe_grouped.hpp", "kernels/linear_q4.hpp", "kernels/swiglu.hpp",
               "kernels/linear_q8.hpp", "kernels/linear.hpp", "kernels/hc.hpp"]
# reference declarations in those headers this library does not define (none)
NOT_BUILT: set = set()

_TYPES = {"int64_t": "long", "int32_t": "int", "uint32_t": "unsigned int", "uint16_t": "unsigned short",
          "uint8_t": "unsigned char", "size_t": "unsigned long", "hipStream_t": "ihipStream_t*",
          "Act": "strix::kernels::Act", "MoeMath": "strix::kernels::MoeMath",
          "MoeSharedAdd": "strix::kernels::MoeSharedAdd", "Q4DeviceView": "strix::Q4DeviceView",
          "Q5DeviceView": "strix::Q5DeviceView", "Q8DeviceView": "strix::Q8DeviceView",
          "Q4ChunkMajorView": "strix::Q4ChunkMajorView", "Q8ChunkMajorView": "strix::Q8ChunkMajorView"}


def _demangled_param(p: str) -> str:
    """One C++ parameter declaration as c++filt prints its type ('const void *x' -> 'void const*')."""
    p = re.sub(r"=.*$", "", p).strip()
    arr = p.endswith("]")
    p = re.sub(r"\[[^\]]*\]$", "", p).strip()
    m = re.match(r"^(const\s+)?([A-Za-z_][\w:]*)\s*([*&]*)\s*[A-Za-z_]\w*$", p)
    assert m, p
    base = _TYPES.get(m.group(2), m.group(2))
    out = base + (" const" if m.group(1) else "")
    ptr = m.group(3) + ("*" if arr else "")
    return out + ptr if ptr else out


def reference_declarations():
    """(name, demangled signature) of every function declared in strix::kernels by the reference headers this
    library replaces."""
    decls = []
    for h in REF_HEADERS:
        src = open(os.path.join(REF, h)).read()
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\n(?:void|size_t|bool)\s+(\w+)\(([^;{]*?)\)\s*;", src):
            params = [p for p in re.split(r",\s*", " ".join(m.group(2).split())) if p]
            sig = f"strix::kernels::{m.group(1)}({', '.join(_demangled_param(p) for p in params)})"
            decls.append((m.group(1), sig))
    return decls


@pytest.mark.skipif(not os.path.isdir(REF), reason="needs the reference's kernel headers under /root/reference, which exist only in the build container (the GPU box has no copy); the CPU suite runs it there")
def test_exports_match_reference_declarations():
    """Every launcher the reference's kernel headers declare (kernels/moe_router, moe_grouped, linear_q4, swiglu,
    linear_q8, linear, hc .hpp) is exported with the same demangled C++ signature, so strixite's call sites link against
    this library with their own headers; and the library exports no act_name (strixite's kernels/norm.hip defines
    it)."""
    import subprocess

    from strixite_amd import _lib

    nm = subprocess.run(["nm", "-DC", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                        check=True).stdout
    exported = {line.split(" ", 2)[2] for line in nm.splitlines() if " T " in line}
    decls = reference_declarations()
    assert len(decls) >= 25
    missing = [sig for name, sig in decls if name not in NOT_BUILT and sig not in exported]
    assert not missing, missing
    assert not any("act_name" in e for e in exported)


def test_strixw_exports_reference_names():
    """The strixw reader / writer / loader export the names strixite formats/strixw.hpp and runtime/strixw_loader.hpp
    declare (the Device placement's subset of StrixwDevice), so the engine's loading code links unchanged."""
    import subprocess

    from strixite_amd import _lib

    nm = subprocess.run(["nm", "-DC", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                        check=True).stdout
    exported = [line.split(" ", 2)[2] for line in nm.splitlines() if " T " in line or " W " in line]
    for name in ["strix::strixw_encoding_name", "strix::strixw_role_name", "strix::strixw_components",
                 "strix::strix_hash64", "strix::StrixHasher::StrixHasher", "strix::StrixHasher::update",
                 "strix::StrixHasher::final", "strix::StrixwTensor::numel", "strix::StrixwTensor::bytes",
                 "strix::StrixwWriter::StrixwWriter", "strix::StrixwWriter::write", "strix::StrixwWriter::finish",
                 "strix::StrixwFile::StrixwFile", "strix::StrixwFile::meta", "strix::StrixwFile::find",
                 "strix::StrixwFile::get", "strix::StrixwFile::data", "strix::StrixwFile::verify_hashes",
                 "strix::StrixwDevice::StrixwDevice", "strix::StrixwDevice::tensor", "strix::StrixwDevice::ptr",
                 "strix::StrixwDevice::q4", "strix::StrixwDevice::q8", "strix::StrixwDevice::f32",
                 "strix::StrixwDevice::bf16"]:
        assert any(e.startswith(name + "(") for e in exported), name


def test_q5_combine_refuses_partial_overlapping_h():
    """The Q5 grouped combine refuses FP32 partials whose bytes overlap h anywhere, also in the upper half that a
    BF16-sized check would miss (the down projection would overwrite h while still reading it)."""
    from strixite_amd import _lib

    L = _lib.lib()
    buf = (C.c_uint8 * 16384)()
    p = (C.addressof(buf) + 255) // 256 * 256
    E, M, A, N, K = 2, 1, 2, 64, 128
    v = _lib.QView(p, p, p, E * N, K, 32)
    ws = p + 4096
    partial = p + 8192                    # M A N floats = 512 bytes
    h = partial + 384                     # inside partial's upper half
    y = p + 12288
    rc = L.strix_linear_q5_experts_combine_grouped(h, C.byref(v), E, p + 2048, p + 2560, ws, 4096, partial, M, A, y,
                                                   1, 0, None, None, 0)
    assert rc == 1 and b"must not overlap" in L.strix_moe_last_error(), L.strix_moe_last_error()
