"""FP32 activations (Act::F32) through the expert and dense projections (strixite kernels/linear_q4.hpp:32-41,
moe_grouped.hpp:3-16: FP32 x against the Q4 / Q8 codes, FP32 accumulation): against float64 closed forms on seeded
data, invalid ids as NaN rows, the shared add in FP32, and the per-slot entry points bit-identical to the grouped
ones (the same per-element arithmetic)."""
import numpy as np
import pytest
import torch

import oracle as orc
from oracle import hc
from strixite_amd import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(*a):
    print("[f32act]", *a, flush=True)


def _rel(got, ref) -> float:
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _weight(bits, N, K, G, seed):
    q, s, m = orc.gen_q(bits, orc.tensor_key(seed, "gu_q"), orc.tensor_key(seed, "gu_s"), N, K, G)
    return moe.QWeight.from_host(bits, q, s, m, N, K, G), hc.weights64(bits, q, s, m, N, K, G)


def _x(M, K, seed):
    return torch.from_numpy(np.random.default_rng(seed).standard_normal((M, K)).astype(np.float32)).to(DEV)


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("bits,G,M", [(4, 64, 1), (4, 128, 37), (8, 32, 5), (8, 64, 130)])
def test_dense_f32_activations(bits, G, M):
    say("dense", bits, G, M)
    w, w64 = _weight(bits, 96, 256, G, 3)
    x = _x(M, 256, M)
    ref = _np(x) @ w64.T
    lin = moe.linear_q4 if bits == 4 else moe.linear_q8
    # FP32 sums of code * x with the min term folded per chunk: rounding relative to the row's largest terms
    assert _rel(_np(lin(x, w, out_dtype=torch.float32)), ref) < 1e-4
    assert _rel(_np(lin(x, w, out_dtype=torch.bfloat16)), ref) < 2.0 ** -7


@pytest.mark.parametrize("bits,G", [(4, 128), (8, 64)])
def test_grouped_and_perslot_f32_activations(bits, G):
    say("experts", bits, G)
    M, A, E, H, I = 5, 3, 8, 256, 64
    gu, gu64 = _weight(bits, E * 2 * I, H, G, 4)
    dn, dn64 = _weight(bits, E * H, I, min(G, I), 5)
    x = _x(M, H, 9)
    ids = np.stack([np.random.default_rng(m).permutation(E)[:A] for m in range(M)]).astype(np.int32)
    ids[3, 1] = -1  # an invalid id: NaN row for its slot, NaN output for its token
    tid = torch.from_numpy(ids).to(DEV)
    ws, _ = moe.moe_group_routes(tid, E)
    h = moe.experts_gather_grouped_swiglu(x, gu, E, ws, M, A)
    torch.cuda.synchronize()
    assert h.dtype == torch.float32
    hn = _np(h)
    X = _np(x)
    good = [s for s in range(M * A) if ids.flat[s] >= 0]
    bad = [s for s in range(M * A) if ids.flat[s] < 0]
    href = np.zeros((M * A, I))
    for s in good:
        e = ids.flat[s]
        g = X[s // A] @ gu64[e * 2 * I:e * 2 * I + I].T
        u = X[s // A] @ gu64[e * 2 * I + I:(e + 1) * 2 * I].T
        href[s] = g / (1 + np.exp(-g)) * u
    assert np.all(np.isnan(hn[bad]))
    assert _rel(hn[good], href[good]) < 1e-4
    coef = np.random.default_rng(2).random((M, A)).astype(np.float32)
    tc = torch.from_numpy(coef).to(DEV)
    hz = h.clone()
    hz[bad] = 0
    s = _x(M, H, 11)
    gl = torch.from_numpy(np.random.default_rng(3).standard_normal((M, 1)).astype(np.float32)).to(DEV)
    err = moe.zero_err()
    y = moe.experts_combine_grouped(hz, dn, E, tid, tc, ws, M, A,
                                    shared={"s": s, "gate_logit": gl, "gate_ld": 1, "gate_index": 0, "err": err})
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    Hz = _np(hz)
    yref = np.zeros((M, H))
    for m in range(M):
        for a in range(A):
            e = ids[m, a]
            if e >= 0:
                yref[m] += coef[m, a] * (Hz[m * A + a] @ dn64[e * H:(e + 1) * H].T)
        yref[m] += _np(s)[m] / (1 + np.exp(-_np(gl)[m, 0]))
    yn = _np(y)
    assert np.all(np.isnan(yn[3])) and not np.any(np.isnan(np.delete(yn, 3, axis=0)))
    assert _rel(np.delete(yn, 3, axis=0), np.delete(yref, 3, axis=0)) < 1e-4
    if bits == 4:  # the per-slot entry points (Q4 in the reference's interface): the same bits as the grouped ones
        e2 = moe.zero_err()
        hp = moe.experts_gather(x, gu, E, tid, e2, swiglu=True)
        assert torch.equal(torch.nan_to_num(hp, nan=7.0), torch.nan_to_num(h, nan=7.0))
        assert to_err(e2) == [1, 0xFFFFFFFF, 3 * A + 1]
        gp = moe.experts_gather(x, gu, E, tid, moe.zero_err())
        gg = moe.experts_gather_grouped(x, gu, E, ws, M, A)
        assert torch.equal(torch.nan_to_num(gp, nan=7.0), torch.nan_to_num(gg, nan=7.0))
        yp = moe.experts_combine(hz, dn, E, tid, tc, moe.zero_err())
        yg = moe.experts_combine_grouped(hz, dn, E, tid, tc, ws, M, A)
        assert torch.equal(torch.nan_to_num(yp, nan=7.0), torch.nan_to_num(yg, nan=7.0))


def to_err(e: torch.Tensor):
    return [int(v) for v in e.cpu().numpy().astype(np.uint32)[:3]]
