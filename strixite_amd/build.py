"""Builds libstrixite_moe.so in-tree: every HIP / C++ source under csrc/ compiled for gfx950 with hipcc, linked
into one shared library next to this file (so it travels with the repository snapshot)."""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libstrixite_moe.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-std=c++20", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
    # packed FP32 instructions stay out of the device code (hipcc's host pass warns that it ignores the feature)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


# hipBLASLt: the prefill router's approximate pass (a plain bf16 GEMM)
LIBS = ["-lhipblaslt"]


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str) -> str:
    obj = os.path.join(OUT, src + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    noise = [l for l in r.stderr.splitlines() if l.strip() and "packed-fp32-ops" not in l]
    if noise:
        print(f"[build] {src}:\n" + "\n".join(noise), file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(OUT, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs, *LIBS], capture_output=True,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


# Host-code sanitizer build: every source's host code compiled with AddressSanitizer and UBSan (the CPU tests never
# launch a kernel), linked into libstrixite_moe_asan.so beside the real library. Load it with
# STRIX_MOE_LIB pointing at it and the clang ASan runtime preloaded (tests/test_zy_sanitizers.py does both).
OUT_ASAN = os.path.join(HERE, "_build_asan")
LIB_ASAN = os.path.join(HERE, "libstrixite_moe_asan.so")
# (the device code is compiled as usual, at -O1, so the library links whole; the sanitizer options apply to the host
# pass only: -Xarch_host before each)
ASAN_FLAGS = ["-std=c++20", "-O1", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Xarch_host", "-g", "-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-sanitize-recover=all",
              "-Xarch_host", "-fno-omit-frame-pointer", "-I", os.path.join(ROOT, "include"), "-I", CSRC]


def asan_runtime() -> str:
    r = subprocess.run([HIPCC, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True,
                       check=True)
    return r.stdout.strip()


def _newest_source() -> float:
    files = [os.path.join(CSRC, f) for f in os.listdir(CSRC)]
    inc = os.path.join(ROOT, "include")
    files += [os.path.join(inc, f) for f in os.listdir(inc)]
    return max(os.path.getmtime(f) for f in files)


def build_asan(jobs: int | None = None, force: bool = False) -> str:
    """Builds libstrixite_moe_asan.so unless it is newer than every source and header (force: always)."""
    if not force and os.path.exists(LIB_ASAN) and os.path.getmtime(LIB_ASAN) > _newest_source():
        return LIB_ASAN
    os.makedirs(OUT_ASAN, exist_ok=True)

    def one(src: str) -> str:
        obj = os.path.join(OUT_ASAN, src + ".o")
        r = subprocess.run([HIPCC, *ASAN_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj], capture_output=True,
                           text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc (sanitizer build) failed on {src}:\n{r.stderr}")
        return obj

    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        objs = list(ex.map(one, srcs))
    tmp = LIB_ASAN + ".tmp"
    r = subprocess.run([HIPCC, "-shared", "-fsanitize=address,undefined", "-shared-libsan", "-fno-gpu-sanitize",
                        f"--offload-arch={ARCH}",
                        "-o", tmp, *objs, *LIBS], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link (sanitizer build) failed:\n{r.stderr}")
    os.replace(tmp, LIB_ASAN)
    return LIB_ASAN


if __name__ == "__main__":
    print(build_asan() if "--asan" in sys.argv else build())
