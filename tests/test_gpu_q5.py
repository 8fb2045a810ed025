"""Q5 experts (strixite formats/q5.hpp; kernels/moe_grouped.hpp:93-104, linear_q4.hpp:47-58) on the GPU: weights
quantized by the oracle's restatement of the reference quantizer (pinned bit for bit by tests/golden/q5.npz), BF16
and FP32 activations against float64 closed forms, invalid ids as NaN rows, the shared add, and the per-slot entry
points bit-identical to the grouped ones."""
import numpy as np
import pytest
import torch

from oracle import q5
from strixite_amd import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[q5]", *a, flush=True)


def _rel(got, ref) -> float:
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _weight(N, K, G, seed):
    w = (np.random.default_rng(seed).standard_normal((N, K)) * 0.05).astype(np.float32)
    q, s, m = q5.quantize(w, G)
    return moe.QWeight.from_host(5, q, s, m, N, K, G), q5.weights64(q, s, m, N, K, G)


@pytest.mark.parametrize("act,G", [("bf16", 128), ("f32", 64), ("bf16", 32)])
def test_q5_experts(act, G):
    say("q5 experts", act, G)
    M, A, E, H, I = 6, 3, 8, 256, 128
    gu, gu64 = _weight(E * 2 * I, H, G, 1)
    dn, dn64 = _weight(E * H, I, G, 2)
    dt = torch.bfloat16 if act == "bf16" else torch.float32
    x = torch.from_numpy(np.random.default_rng(3).standard_normal((M, H)).astype(np.float32)).to(DEV).to(dt)
    ids = np.stack([np.random.default_rng(m).permutation(E)[:A] for m in range(M)]).astype(np.int32)
    ids[4, 2] = E  # an invalid id
    tid = torch.from_numpy(ids).to(DEV)
    ws, _ = moe.moe_group_routes(tid, E)
    h = moe.experts_gather_grouped_swiglu(x, gu, E, ws, M, A)
    torch.cuda.synchronize()
    assert h.dtype == dt
    X = _np(x)
    good = [s for s in range(M * A) if ids.flat[s] < E]
    bad = [s for s in range(M * A) if ids.flat[s] >= E]
    href = np.zeros((M * A, I))
    for s in good:
        e = ids.flat[s]
        g = X[s // A] @ gu64[e * 2 * I:e * 2 * I + I].T
        u = X[s // A] @ gu64[e * 2 * I + I:(e + 1) * 2 * I].T
        href[s] = g / (1 + np.exp(-g)) * u
    hn = _np(h)
    tol = 2.0 ** -7 if act == "bf16" else 1e-4
    assert np.all(np.isnan(hn[bad])) and _rel(hn[good], href[good]) < tol
    hz = h.clone()
    hz[bad] = 0
    coef = np.random.default_rng(4).random((M, A)).astype(np.float32)
    tc = torch.from_numpy(coef).to(DEV)
    s = torch.from_numpy(np.random.default_rng(5).standard_normal((M, H)).astype(np.float32)).to(DEV).to(dt)
    gl = torch.from_numpy(np.random.default_rng(6).standard_normal((M, 1)).astype(np.float32)).to(DEV)
    y = moe.experts_combine_grouped(hz, dn, E, tid, tc, ws, M, A,
                                    shared={"s": s, "gate_logit": gl, "gate_ld": 1, "gate_index": 0,
                                            "err": moe.zero_err()})
    torch.cuda.synchronize()
    Hz = _np(hz)
    yref = np.zeros((M, H))
    for m in range(M):
        for a in range(A):
            if ids[m, a] < E:
                yref[m] += coef[m, a] * (Hz[m * A + a] @ dn64[ids[m, a] * H:(ids[m, a] + 1) * H].T)
        yref[m] += _np(s)[m] / (1 + np.exp(-_np(gl)[m, 0]))
    yn = _np(y)
    assert np.all(np.isnan(yn[4]))
    ok = [m for m in range(M) if m != 4]
    assert _rel(yn[ok], yref[ok]) < tol
    # per-slot entry points: the same per-element arithmetic as the grouped ones
    err = moe.zero_err()
    hp = moe.experts_gather(x, gu, E, tid, err, swiglu=True)
    assert torch.equal(torch.nan_to_num(hp.float(), nan=7.0), torch.nan_to_num(h.float(), nan=7.0))
    assert [int(v) for v in err.cpu().numpy().astype(np.uint32)] == [1, E, 4 * A + 2]
    gp = moe.experts_gather(x, gu, E, tid, moe.zero_err())
    gg = moe.experts_gather_grouped(x, gu, E, ws, M, A)
    assert torch.equal(torch.nan_to_num(gp.float(), nan=7.0), torch.nan_to_num(gg.float(), nan=7.0))
    yp = moe.experts_combine(hz, dn, E, tid, tc, moe.zero_err())
    yg = moe.experts_combine_grouped(hz, dn, E, tid, tc, ws, M, A)
    assert torch.equal(torch.nan_to_num(yp.float(), nan=7.0), torch.nan_to_num(yg.float(), nan=7.0))


def test_q5_refuses_f16_h():
    say("q5 refusals")
    M, A, E, H, I = 2, 2, 4, 256, 128
    gu, _ = _weight(E * 2 * I, H, 128, 1)
    x = torch.zeros((M, H), dtype=torch.bfloat16, device=DEV)
    tid = torch.from_numpy(np.array([[0, 1], [2, 3]], np.int32)).to(DEV)
    ws, _ = moe.moe_group_routes(tid, E)
    with pytest.raises(RuntimeError, match="F16 h form"):
        moe.experts_gather_grouped_swiglu(x, gu, E, ws, M, A, h_f16=True)
