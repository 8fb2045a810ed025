"""moe_layer_forward_noalloc (C-ABI strix_moe_layer_forward_noalloc): the sublayer on the library's fixed device
scratch array, no workspace argument. Its outputs equal moe_layer_forward's (the same kernels on a caller-owned
workspace) bit for bit, over two calls in a row on one device, the second with fewer tokens (the array still holds
the first call's tables and partials)."""
import ctypes as C
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from strixite_amd import _lib as L  # noqa: E402
from strixite_amd import moe  # noqa: E402


def say(*a):
    print("[gpu]", *a, file=sys.stderr, flush=True)


def _outputs(M, H, k, dev="cuda"):
    return {"y": torch.full((M, H), 7.0, dtype=torch.bfloat16, device=dev),
            "x_out": torch.full((M, H), 7.0, dtype=torch.bfloat16, device=dev),
            "ids": torch.full((M, k), -5, dtype=torch.int32, device=dev),
            "coef": torch.full((M, k), 9.0, dtype=torch.float32, device=dev),
            "err": torch.zeros(6, dtype=torch.int32, device=dev)}


def _noalloc(layer, x, out):
    p = moe._p
    L.check(L.lib().strix_moe_layer_forward_noalloc(C.byref(layer._w), p(x), x.shape[0], None, p(out["y"]),
                                                    p(out["x_out"]), p(out["ids"]), p(out["coef"]), p(out["err"]),
                                                    moe._stream()))


def test_noalloc_matches_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    H, E, k, I = 3072, 512, 10, 512
    layer = moe.MoeLayer.synth(H, E, k, I, seed=0, layer=2)
    cap = L.lib().strix_moe_layer_noalloc_max_bytes()
    assert cap == 16 << 20
    # the largest batch that fits the array, then a smaller one
    big = max(M for M in range(1, 257) if layer.workspace_bytes(M) <= cap)
    assert big >= 16, big
    for M, seed in ((big, 31), (5, 32)):
        say("noalloc", M)
        x = moe.synth_bf16_normal(seed, "x", 0, (M, H), 1.0)
        ref = layer.forward(x)
        got = _outputs(M, H, k)
        _noalloc(layer, x, got)
        torch.cuda.synchronize()
        for name in ("ids", "coef", "y", "x_out", "err"):
            assert torch.equal(got[name], ref[name]), (M, name)
        assert int(got["err"][0]) == 0 and int(got["err"][3]) == 0
    # a batch the array cannot hold is refused before any launch
    M = big + 1
    x = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(moe.StrixError, match="more than the fixed"):
        _noalloc(layer, x, _outputs(M, H, k))
