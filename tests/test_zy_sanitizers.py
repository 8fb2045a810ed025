"""Host code under AddressSanitizer and UBSan (CPU only): the library's sources compiled for the host with
-fsanitize=address,undefined (strixite_amd/build.py build_asan; no device code, no kernel launched) and the C oracle
likewise (oracle/Makefile target asan), then the strixw reader / writer tests (corruption cases included), the
boundary's precondition and error-word tests and the oracle tests run in a child pytest with the sanitizer runtime
preloaded. Any sanitizer report aborts the child (-fno-sanitize-recover=all), so the child's exit status is the
verdict."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SUITES = ["tests/test_strixw.py", "tests/test_boundary.py", "tests/test_oracle.py", "tests/test_hc_oracle.py",
          "tests/test_q5_oracle.py"]


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") or shutil.which("make") is None,
                    reason="needs hipcc and make for the sanitizer builds")
def test_host_code_under_asan_and_ubsan():
    sys.path.insert(0, ROOT)
    from strixite_amd import build as b

    lib = b.build_asan()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": b.asan_runtime(),
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1",  # the interpreter itself is not leak-clean
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "STRIX_MOE_LIB": lib,
        "ORACLE_LIB": os.path.join(ROOT, "oracle", "liboracle_moe_asan.so"),
    })
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *SUITES],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, tail
    assert " passed" in r.stdout, tail
    # the sanitizer is live: a read one byte past a 64-byte heap buffer inside the library's hash is reported
    probe = ("import ctypes as C, numpy as np\n"
             "from strixite_amd import _lib as L\n"
             "a = np.zeros(64, np.uint8)\n"
             "L.lib().strix_strixw_hash64.restype = C.c_uint64\n"
             "L.lib().strix_strixw_hash64(C.c_void_p(a.ctypes.data), C.c_size_t(65))\n")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr, r.stderr[-2000:]
