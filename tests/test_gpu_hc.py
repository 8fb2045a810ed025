"""The hyper-connection mix (hc_mix_down, hc_mix_up; strixite kernels/hc.hpp:31-50) on the GPU through the C-ABI,
against the float64 oracle (oracle/hc.py) on seeded inputs: Q4 and Q8 weights, BF16 and F32 streams, token counts
across the kernels' token groups, the inject and no-inject forms, and the refusals of the reference's preconditions."""
import numpy as np
import pytest
import torch

import oracle as orc
from oracle import hc
from strixite_amd import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[hc]", *a, flush=True)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().astype(np.float64)


def _rel(got, ref) -> float:
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _weight(bits, N, K, G, seed, chunk_major=False):
    q, s, m = orc.gen_q(bits, orc.tensor_key(seed, "gu_q"), orc.tensor_key(seed, "gu_s"), N, K, G)
    w64 = hc.weights64(bits, q, s, m, N, K, G)
    if chunk_major:
        q, s, m = hc.to_chunk_major(bits, q, s, m, N, K, G)
    return moe.QWeight.from_host(bits, q, s, m, N, K, G), w64


# token counts below 256 (and d % 128 != 0) take the vector-row down kernel, the rest the matrix-core tiles; every up
# mix runs on the matrix cores (16-token tiles up to 16 tokens, 32-token tiles above)
CASES = [(4, 64, "bf16", 1, 256, 64, True), (4, 128, "f32", 5, 256, 96, True), (8, 32, "bf16", 37, 128, 32, False),
         (8, 64, "f32", 8, 512, 320, True), (4, 64, "bf16", 3, 2560, 320, True), (4, 32, "f32", 40, 256, 320, True),
         (8, 128, "bf16", 100, 384, 64, True), (8, 32, "f32", 17, 128, 96, False), (4, 64, "bf16", 16, 160, 64, True),
         (8, 128, "bf16", 300, 384, 64, True), (4, 32, "f32", 260, 256, 320, True), (8, 32, "f32", 256, 128, 96, False),
         (4, 64, "bf16", 257, 160, 64, True), (4, 64, "bf16", 4096, 2560, 320, True)]


@pytest.mark.parametrize("bits,G,act,T,d,r,inject", CASES)
def test_hc_mix_matches_oracle(bits, G, act, T, d, r, inject):
    say("mix", bits, G, act, T, d, r, inject)
    dt = torch.bfloat16 if act == "bf16" else torch.float32
    x = torch.from_numpy(np.random.default_rng(T).standard_normal((T, 4 * d)).astype(np.float32)).to(DEV).to(dt)
    R = r + (4 if inject else 0)
    w, w64 = _weight(bits, R, 4 * d, G, 21)
    h, w_in, inv = moe.hc_mix_down(x, w, r, inject, 1e-6)
    torch.cuda.synchronize()
    # the float64 oracle on every token up to 256, else on 64 spread tokens and the last (each token is independent)
    rows = np.arange(T) if T <= 256 else np.unique(np.append(np.linspace(0, T - 1, 64).astype(np.int64), T - 1))
    xs = _np(x)[rows]
    hr, wir, invr = hc.hc_mix_down(xs, w64, d, r, inject, 1e-6)
    assert _rel(_np(inv)[rows], invr) < 1e-5
    assert _rel(_np(h)[rows], hr) < 1e-4
    if inject:
        assert _rel(_np(w_in)[rows], wir) < 1e-5
    # the up projection from the kernel's own h and inv (so its check does not inherit the down's FP32 rounding)
    Gu = 32 if r % 64 else 64
    wu, wu64 = _weight(bits, 4 * d, r, Gu, 22, chunk_major=True)
    nw = torch.from_numpy(np.random.default_rng(5).standard_normal(4 * d).astype(np.float32) * 0.1).to(DEV)
    u = moe.hc_mix_up(h, wu, x, nw, inv)
    torch.cuda.synchronize()
    ur = hc.hc_mix_up(_np(h)[rows], wu64, xs, _np(nw), _np(inv)[rows], d)
    assert u.dtype == dt
    # F32: each chunk's s * sum(h * code) and m * sum(h) nearly cancel (Q8: m = -128 s), so FP32 rounding of those
    # terms shows at ~1e-5 of the result
    assert _rel(_np(u)[rows], ur) < (2.0 ** -8 if act == "bf16" else 1e-4)


def test_hc_mix_refusals():
    say("refusals")
    x = torch.zeros((2, 4 * 64), dtype=torch.bfloat16, device=DEV)
    w, _ = _weight(4, 8 + 4, 4 * 64, 64, 1)
    with pytest.raises(RuntimeError, match="go with inject = true"):
        h = torch.empty((2, 8), device=DEV)
        inv = torch.empty((2, 4), device=DEV)
        from strixite_amd import _lib as L
        import ctypes as C
        v = w.view()
        L.check(L.lib().strix_hc_mix_down(x.data_ptr(), C.byref(v), 4, 2, 4, 64, 8, 1, 1e-6, h.data_ptr(), None,
                                          inv.data_ptr(), 1, None))
    with pytest.raises(RuntimeError, match="rows are needed"):
        moe.hc_mix_down(x, w, 8, False, 1e-6)  # 12 rows given for r = 8 without the injection rows
