"""strixw loaded into HBM (StrixwDevice) on the GPU: every component's device bytes equal the file's, and the MoE
sublayers built from the reference-written fixture match the oracle run on the same file's weights."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

import oracle as orc
import oracle.strixw as ostrixw
from gpu_util import rel_err, to_np
from strixite_amd import moe, strixw

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "layers.strixw")
LM = "model.language_model.layers."


def say(*a):
    print("[strixw]", *a, flush=True)


def device_bytes(ptr: int, n: int) -> np.ndarray:
    """n bytes at a device address, copied to the host with the process's HIP runtime (hipMemcpy D2H)."""
    torch.cuda.synchronize()
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    out = np.empty(n, np.uint8)
    assert hip.hipMemcpy(out.ctypes.data, ptr, n, 2) == 0
    return out


def test_device_load_fixture_bytes():
    say("load fixture")
    d = strixw.StrixwDevice(FIXTURE, 3)
    o = ostrixw.File(FIXTURE)
    assert d.device_bytes == len(o.buf) - o.data_offset
    for t in o.tensors:
        for role, off, nb, _ in t["components"]:
            p = d.ptr(t["name"], role)
            assert p % 256 == 0
            assert np.array_equal(device_bytes(p, nb), np.frombuffer(o.buf, np.uint8, nb, off)), (t["name"], role)


@pytest.mark.parametrize("layer,M", [(0, 5), (0, 40), (1, 5), (1, 40)])
def test_layer_from_fixture_matches_oracle(layer, M):
    """Layer 0: the shared expert stacked as expert E (Q4 G128); layer 1: Q8 G64 routed experts with a separate Q8
    shared expert. Routing bit-exact, output within 1e-2 of the oracle on the file's own weights."""
    say("layer", layer, "M", M)
    d = strixw.StrixwDevice(FIXTURE, 2)
    L = d.moe_layer(f"{LM}{layer}.", 2)
    assert L.shared_stacked == (layer == 0) and L.has_shared == (layer == 1)
    x = moe.synth_bf16_normal(20 + layer, "x", M, (M, 128), 1.0)
    out = L.forward(x)
    torch.cuda.synchronize()
    w = ostrixw.File(FIXTURE).moe_layer(f"{LM}{layer}.", 2)
    o = orc.moe_layer(w, to_np(x))
    assert np.array_equal(to_np(out["ids"]), o["ids"])
    assert np.allclose(to_np(out["coef"]), o["coef"], rtol=2e-6, atol=1e-7)
    assert rel_err(to_np(out["y"]), o["y"]) < 1e-2
    assert rel_err(to_np(out["x_out"]), o["out"]) < 1e-2
    assert not to_np(out["err"]).any()


def test_large_file_load_many_chunks(tmp_path):
    """A 300 MB file (five 64 MiB chunks and a partial one over four workers) arrives whole: the device copy of the
    region equals the file's bytes."""
    say("large file")
    rng = np.random.default_rng(1)
    N, K = 4 * 1024 * 1024 + 16, 128  # q4: N K / 2 bytes of codes
    q = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    s = rng.integers(0, 65536, N, dtype=np.uint16)
    p = str(tmp_path / "big.strixw")
    strixw.write(p, {"kind": "test"}, [
        {"name": "small", "encoding": "f32", "shape": [5], "data": {"data": np.arange(5, dtype=np.float32)}},
        {"name": "big", "encoding": "q4", "shape": [N, K], "group_size": 128,
         "data": {"q": q, "scale": s, "min": s[::-1].copy()}}])
    d = strixw.StrixwDevice(p, 4)
    f = strixw.StrixwFile(p)
    region = device_bytes(d.ptr("small"), d.device_bytes)
    buf = np.fromfile(p, np.uint8)[f.data_offset:]
    assert region.size == buf.size and np.array_equal(region, buf)
    assert d.load_seconds > 0
