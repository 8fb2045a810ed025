"""Parity of the gfx950 HIP path against the CPU oracle, through the C-ABI (strixite_amd.moe forwards to it).

Bars: bit-exact for integer / index work and for the router logits (one specified FP32 order); for the expert math
max|got - ref| / max|ref| <= 1e-2 in bf16 (BASELINE's layer tolerance), with tighter bounds where the f16 weight
rounding allows. Sizes keep the oracle to seconds; the full-size configs check the routing on every token and the
layer output on a seeded subset of tokens (the layer is token-independent once routed).
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as orc  # noqa: E402
from gpu_util import balanced, oracle_weights, qspec, rel_err, to_np, zipf_bias  # noqa: E402
from strixite_amd import moe  # noqa: E402

DEV = "cuda"


def say(*a):
    print("[gpu]", *a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    moe.L.lib()  # loud failure if the library is missing
    yield
    torch.cuda.synchronize()


def bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)


# ---- generator --------------------------------------------------------------------------------------------------
def test_synth_matches_host_generator():
    say("synth")
    x = moe.synth_bf16_normal(7, "x", 3, (5, 1000), 1.0)
    ref = orc.gen_bf16_normal(orc.tensor_key(7, "x", 3), 1.0, (5, 1000))
    assert np.array_equal(to_np(x), ref)
    for bits, G in ((4, 128), (8, 64)):
        w = moe.QWeight.synth(bits, 7, "gu_q", "gu_s", 2, 48, 512, G)
        q, s, m = orc.gen_q(bits, orc.tensor_key(7, "gu_q", 2), orc.tensor_key(7, "gu_s", 2), 48, 512, G)
        assert np.array_equal(to_np(w.q), q) and np.array_equal(to_np(w.scale), s) and np.array_equal(to_np(w.minv), m)
    u = moe.synth_uniform_pm1(7, "logits", 0, (3, 513))
    assert np.array_equal(to_np(u), orc.gen_uniform_pm1(orc.tensor_key(7, "logits", 0), (3, 513)))


# ---- router -----------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 65, 2048), (16, 513, 3072), (5, 7, 1000), (37, 129, 512), (300, 513, 3072),
                                   (257, 70, 512), (7, 30, 4096), (64, 513, 2048), (3, 17, 3072)])
def test_linear_bf16w_bit_exact(M, N, K):
    say("linear_bf16w", M, N, K)
    x = orc.gen_bf16_normal(orc.tensor_key(1, "x"), 1.0, (M, K))
    w = orc.gen_bf16_normal(orc.tensor_key(1, "router"), 0.02, (N, K))
    y = moe.linear_bf16w(bf16(x), bf16(w))
    ref = orc.router_logits(x, w)
    assert np.array_equal(to_np(y).view(np.uint32), ref.view(np.uint32))
    yb = moe.linear_bf16w(bf16(x), bf16(w), out_dtype=torch.bfloat16)
    assert np.array_equal(to_np(yb), orc.f32_to_bf16(ref))
    # Act::F32 activations: an FP32 x holding the same BF16 values gives the same bits (same products, same order)
    xf = torch.from_numpy(orc.bf16_to_f32(x)).to(DEV)
    yf = moe.linear_bf16w(xf, bf16(w))
    assert np.array_equal(to_np(yf).view(np.uint32), ref.view(np.uint32))
    # and general FP32 x against the float64 sum, within the FP32 summation bound (2 K u |x| |w| per dot)
    xg = torch.from_numpy(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32)).to(DEV)
    yg = to_np(moe.linear_bf16w(xg, bf16(w))).astype(np.float64)
    w64 = orc.bf16_to_f32(w).astype(np.float64)
    x64 = xg.cpu().numpy().astype(np.float64)
    bound = 2 * K * 2.0 ** -24 * np.abs(x64) @ np.abs(w64).T + 1e-30
    assert np.all(np.abs(yg - x64 @ w64.T) <= bound)


@pytest.mark.parametrize("E,k", [(64, 8), (512, 10), (1024, 32), (100, 32), (7, 7)])
def test_moe_router_matches_oracle(E, k):
    say("moe_router", E, k)
    rng = np.random.default_rng(E * 100 + k)
    M = 300
    lg = rng.standard_normal((M, E + 3)).astype(np.float32)
    lg[5, :] = 0.25  # all equal: ids 0..k-1
    lg[6, 3:9] = lg[6, :E].max() + 1  # a tie at the top
    lg[7, : E // 2] = lg[7, E // 2: 2 * (E // 2)]  # pairwise ties everywhere
    lg[8, :] = 0.0
    lg[8, 1::2] = -0.0  # -0 and +0 compare equal: the lower index wins
    lg[9, :] = -1.0
    lg[9, E - 1] = lg[9, E // 2] = 3.0  # a tie between far-apart experts
    # equal values straddling the k-th place (the candidate picks rank them by index): a few above, then 40 equal
    # (at most 64 candidates), then 80 equal (more than 64: the rounds)
    for r, n_eq in ((10, 40), (11, 80)):
        lg[r, :] = -2.0
        top = min(k - 1, 3)
        lg[r, E - top:E] = 5.0
        eq = rng.permutation(E - top)[:min(n_eq, E - top)]
        lg[r, eq] = 1.0
    ids, coef, err = moe.moe_router(torch.from_numpy(lg).to(DEV), E, k, ld=E + 3)
    rids, rcoef, rerr = orc.topk(lg, E, k)
    assert np.array_equal(to_np(ids), rids)
    assert np.allclose(to_np(coef), rcoef, rtol=2e-6, atol=1e-7)
    assert to_np(err)[0] == 0 and rerr[0] == 0
    # bf16 logits
    lb = orc.f32_to_bf16(lg)
    ids_b, coef_b, _ = moe.moe_router(bf16(lb), E, k, ld=E + 3)
    rids_b, rcoef_b, _ = orc.topk(orc.bf16_to_f32(lb), E, k)
    assert np.array_equal(to_np(ids_b), rids_b)
    assert np.allclose(to_np(coef_b), rcoef_b, rtol=2e-6, atol=1e-7)


def test_moe_router_shared_and_nonfinite():
    say("moe_router nonfinite")
    E, k, M = 512, 10, 64
    lg = np.random.default_rng(3).standard_normal((M, E + 1)).astype(np.float32)
    lg[9, 100] = np.nan
    lg[9, 7] = np.inf
    lg[20, E] = -np.inf
    t = torch.from_numpy(lg).to(DEV)
    ids, coef, err = moe.moe_router(t, E, k, shared_logit=t[:, E:], shared_ld=E + 1, shared_id=E, ld=E + 1)
    rids, rcoef, _ = orc.topk(lg, E, k, shared=np.ascontiguousarray(lg[:, E:]), shared_ld=1, shared_id=E)
    assert np.array_equal(to_np(ids), rids)
    ok = ~np.isnan(rcoef)
    assert np.array_equal(np.isnan(to_np(coef)), ~ok)
    assert np.allclose(to_np(coef)[ok], rcoef[ok], rtol=2e-6, atol=1e-7)
    e = to_np(err).view(np.uint32)
    assert e[0] == 1 and (tuple(e[1:]) in {(9, 7), (20, E)})  # the first flag of either failing token wins
    with pytest.raises(moe.StrixError, match="non-finite router logit"):
        moe.check_router_error(err, "L0 moe")


# ---- packing -----------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,A,E", [(1, 8, 64), (16, 10, 512), (6, 11, 1023), (300, 10, 512), (4096, 10, 512),
                                   (513, 64, 1023), (3, 1, 1)])
def test_group_routes_bit_exact(M, A, E):
    say("group_routes", M, A, E)
    rng = np.random.default_rng(M + A + E)
    ids = rng.integers(0, E, (M, A)).astype(np.int32)
    if M * A > 200:  # Zipf-like skew: one hot bucket
        ids[rng.random((M, A)) < 0.3] = E // 2
    ws, err = moe.moe_group_routes(torch.from_numpy(ids).to(DEV), E)
    t = moe.route_tables(ws, M, A, E)
    off, slots, rerr = orc.group_routes(ids, E)
    assert np.array_equal(to_np(t["offsets"]), off)
    assert np.array_equal(to_np(t["slots"]), slots)
    assert int(t["S"]) == M * A and int(t["E"]) == E
    assert int(t["n_tiles"]) == int(sum((c + 15) // 16 for c in np.diff(off)))
    assert to_np(err)[0] == 0
    _check_pairs(to_np(ws), M * A, E, off)


def _check_pairs(w, S, E, off):
    """The F16 GEMM's 128-slot pairs: every bucket's slots cut into pairs {bucket, first, rows} exactly once, listed
    with their 32-slot sub-tile counts non-increasing. Offsets of the workspace layout (route_small.hpp Layout):
    header 4, offsets E + 2, slots S, 16-slot records of 20 ints, 64-slot records of 4, then the pairs and their
    count."""
    t16 = min(S, S // 16 + E + 2)
    t64 = min(S, S // 64 + E + 2)
    t16_rec = (4 + E + 2 + S + 3) // 4 * 4
    pair_rec = t16_rec + 20 * t16 + 4 * t64
    n = int(w[pair_rec + 4 * t64])
    cnt = np.diff(off)
    want = {(b, int(off[b]) + 128 * q, int(min(128, cnt[b] - 128 * q))) for b in range(E + 1)
            for q in range((int(cnt[b]) + 127) // 128)}
    assert n == len(want)
    recs = w[pair_rec:pair_rec + 4 * n].reshape(n, 4)
    assert {tuple(int(v) for v in r[:3]) for r in recs} == want
    subtiles = (recs[:, 2] + 31) // 32
    assert np.all(np.diff(subtiles) <= 0)


def test_group_routes_invalid_ids():
    say("group_routes invalid")
    for M, A in ((16, 10), (2000, 10)):
        E = 512
        ids = np.random.default_rng(M).integers(0, E, (M, A)).astype(np.int32)
        ids[3, 4], ids[11, 0], ids[12, 9] = -1, E, 99999
        ws, err = moe.moe_group_routes(torch.from_numpy(ids).to(DEV), E)
        off, slots, rerr = orc.group_routes(ids, E)
        t = moe.route_tables(ws, M, A, E)
        assert np.array_equal(to_np(t["offsets"]), off) and np.array_equal(to_np(t["slots"]), slots)
        assert np.array_equal(to_np(err).view(np.uint32), rerr)  # the first invalid slot in slot order
        _check_pairs(to_np(ws), M * A, E, off)
        with pytest.raises(moe.StrixError, match="out of range"):
            moe.check_expert_error(err)


# ---- expert projections ------------------------------------------------------------------------------------------
def _experts(bits, E, H, I, seed=11):
    G = 128 if bits == 4 else 64
    gu = moe.QWeight.synth(bits, seed, "gu_q", "gu_s", 0, E * 2 * I, H, G)
    dn = moe.QWeight.synth(bits, seed, "dn_q", "dn_s", 0, E * H, I, G)
    return gu, dn


def _bf16_partials(pt: torch.Tensor) -> np.ndarray:
    """The F16 math's per-slot partials: BF16 [S, N] in the first half of the FP32 [S, N] partial buffer (the
    reference's layout for its F16 kinds, strixite kernels/moe_grouped.hpp:84)."""
    S, N = pt.shape
    return to_np(pt.view(-1).view(torch.bfloat16)[: S * N].reshape(S, N))


def _expert_gemm_size(S, E):
    """The grouped projections' GEMM kernels take over at S >= 1024 slots and >= 16 slots an expert."""
    return S >= 1024 and S >= 16 * E


@pytest.mark.parametrize("bits,M,A,E,H,I", [(4, 16, 10, 64, 512, 256), (8, 1, 8, 64, 512, 128),
                                            (4, 300, 8, 16, 256, 128), (8, 40, 4, 8, 256, 64)])
def test_grouped_gate_up_swiglu_and_down(bits, M, A, E, H, I):
    say("grouped experts", bits, M, A, E, H, I)
    gu, dn = _experts(bits, E, H, I)
    x = orc.gen_bf16_normal(orc.tensor_key(2, "x"), 1.0, (M, H))
    ids = np.stack([np.random.default_rng(m).permutation(E)[:A] for m in range(M)]).astype(np.int32)
    tid = torch.from_numpy(ids).to(DEV)
    ws, _ = moe.moe_group_routes(tid, E)
    h = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A)
    b, q, s, m, G = qspec(gu)
    href = orc.experts_gate_up_swiglu(x, orc.qview(b, q, s, m, gu.N, H, G), E, ids)
    assert rel_err(to_np(h), href) < 1e-2
    # Q4 under the F16 kinds (the default) runs the reference's F16 math at every batch size (x and the weights
    # rounded to F16): equal to its model up to FP32 summation order and the bf16 rounding of h
    f16 = bits == 4
    if f16:
        h16 = orc.experts_gate_up_swiglu_f16math(x, b, q, s, m, gu.N, H, G, E, ids)
        assert rel_err(to_np(h), h16) < 2.0 ** -8
        # the exact-weight kinds (F32, WmmaBf16) keep their own kernel
        hx = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A, math=moe.MOE_MATH_WMMA_BF16)
        assert rel_err(to_np(hx), href) < 2.0 ** -7
    # the f16-bits form holds the same values wherever they lie in f16's normal range (|v| >= 2^-14)
    hf = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A, h_f16=True)
    normal = h.float().abs() >= 2.0 ** -14
    assert torch.equal(hf.float()[normal], h.float()[normal])
    assert (hf.float() - h.float()).abs().max().item() <= 2.0 ** -24
    coef = np.random.default_rng(5).random((M, A)).astype(np.float32)
    pt = torch.empty((M * A, H), dtype=torch.float32, device=DEV)
    y = moe.experts_combine_grouped(h, dn, E, tid, torch.from_numpy(coef).to(DEV), ws, M, A, partial=pt)
    b, q, s, m, G = qspec(dn)
    part = orc.experts_down(to_np(h), orc.qview(b, q, s, m, dn.N, I, G), E, ids)
    if f16:  # the F16 math's per-slot outputs, stored BF16: its model rounded to BF16, up to FP32 summation order
        pb = _bf16_partials(pt)
        p16 = orc.experts_down_f16math(to_np(h), b, q, s, m, dn.N, I, G, E, ids)
        assert rel_err(pb, orc.f32_to_bf16(p16)) <= 2.0 ** -8
        assert np.mean(pb == orc.f32_to_bf16(p16)) > 0.99
        assert rel_err(pb, part) < 2.0 ** -7
        px = torch.empty_like(pt)
        moe.experts_combine_grouped(h, dn, E, tid, torch.from_numpy(coef).to(DEV), ws, M, A, partial=px,
                                    math=moe.MOE_MATH_WMMA_BF16)
        assert rel_err(px.cpu().numpy(), part) < 1e-4
        part = orc.bf16_to_f32(pb)  # what the F16 combine sums
    else:
        # the per-slot down outputs before any bf16 rounding: fp32 accuracy (Q4's 128 + n codes cancel against m - 128 s)
        assert rel_err(pt.cpu().numpy(), part) < 1e-4
    yref, _ = orc.combine(part, ids, coef, E, H)
    assert rel_err(to_np(y), yref) < 1e-2
    # the f16-h form: under the F16 math its h holds the F16 operands the BF16 h converts to, so y is the same bits;
    # Q8 (exact weights) sums in another order, so an output may round to the neighbouring bf16
    y2 = moe.experts_combine_grouped(hf, dn, E, tid, torch.from_numpy(coef).to(DEV), ws, M, A, h_f16=True)
    if f16:
        assert torch.equal(y2, y)
    else:
        assert rel_err(to_np(y2), to_np(y)) < 2.0 ** -8


def test_grouped_gather_plain_q4():
    say("grouped gather plain")
    M, A, E, H, I = 9, 3, 8, 256, 128
    gu, _ = _experts(4, E, H, I)
    x = orc.gen_bf16_normal(orc.tensor_key(3, "x"), 1.0, (M, H))
    ids = np.random.default_rng(1).integers(0, E, (M, A)).astype(np.int32)
    ws, _ = moe.moe_group_routes(torch.from_numpy(ids).to(DEV), E)
    w = orc.dequantize(4, *qspec(gu)[1:4], gu.N, H, gu.G).astype(np.float64)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    N = 2 * I
    ref = np.stack([w[ids.ravel()[s] * N:(ids.ravel()[s] + 1) * N] @ xf[s // A] for s in range(M * A)])
    # exact weights: FP32 sums rounded once to bf16
    yx = to_np(moe.experts_gather_grouped(bf16(x), gu, E, ws, M, A, math=moe.MOE_MATH_WMMA_BF16))
    assert rel_err(yx, ref) < 2.0 ** -8
    # the F16 kinds: the F16 math's outputs rounded once to bf16, against its model up to FP32 summation order
    y = to_np(moe.experts_gather_grouped(bf16(x), gu, E, ws, M, A))
    b, q, s, m, G = qspec(gu)
    y16 = orc.f32_to_bf16(orc.experts_gather_f16math(x, b, q, s, m, gu.N, H, G, E, ids))
    assert rel_err(y, y16) <= 2.0 ** -8 and np.mean(y == y16) > 0.99
    assert rel_err(y, ref) < 1e-2


def test_stream_kernels_invalid_ids_make_nan_rows():
    """The gathered LDS-ring gate_up and the stream down at M above 16 (exact-weight kinds): a slot with an invalid id
    (-1, E, beyond) gets a NaN h row and NaN partials; the other slots match the oracle."""
    say("stream kernels invalid ids")
    M, A, E, H, I = 48, 4, 32, 3072, 512
    gu, dn = _experts(4, E, H, I, seed=19)
    x = orc.gen_bf16_normal(orc.tensor_key(8, "x"), 1.0, (M, H))
    ids = np.stack([np.random.default_rng(500 + m).permutation(E)[:A] for m in range(M)]).astype(np.int32)
    ids[5, 1], ids[20, 3], ids[47, 0] = -1, E, E + 7
    tid = torch.from_numpy(ids).to(DEV)
    ws, _ = moe.moe_group_routes(tid, E)
    ex = moe.MOE_MATH_WMMA_BF16
    h = to_np(moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A, math=ex))
    bad = np.array([5 * A + 1, 20 * A + 3, 47 * A + 0])
    good = np.setdiff1d(np.arange(M * A), bad)
    assert np.all(np.isnan(orc.bf16_to_f32(h[bad]))) and not np.isnan(orc.bf16_to_f32(h[good])).any()
    ok_ids = ids.copy()
    ok_ids[ids < 0], ok_ids[ids >= E] = 0, 0
    b, q, s, m, G = qspec(gu)
    href = orc.experts_gate_up_swiglu(x, orc.qview(b, q, s, m, gu.N, H, G), E, ok_ids)
    assert rel_err(h[good], href[good]) < 1e-2
    hz = h.copy()
    hz[bad] = 0
    pt = torch.empty((M * A, H), dtype=torch.float32, device=DEV)
    coef = torch.full((M, A), 0.25, device=DEV)
    moe.experts_combine_grouped(torch.from_numpy(hz.view(np.int16)).to(DEV).view(torch.bfloat16), dn, E, tid, coef,
                                ws, M, A, partial=pt, math=ex)
    p = pt.cpu().numpy()
    assert np.all(np.isnan(p[bad]))
    b, q, s, m, G = qspec(dn)
    pref = orc.experts_down(hz, orc.qview(b, q, s, m, dn.N, I, G), E, ok_ids)
    assert rel_err(p[good], pref[good]) < 1e-4


def test_invalid_ids_make_nan_rows():
    say("experts invalid ids")
    M, A, E, H, I = 4, 2, 8, 256, 128
    gu, dn = _experts(4, E, H, I)
    x = orc.gen_bf16_normal(orc.tensor_key(4, "x"), 1.0, (M, H))
    ids = np.array([[0, 1], [2, -1], [3, 4], [5, 8]], np.int32)
    tid = torch.from_numpy(ids).to(DEV)
    ws, err = moe.moe_group_routes(tid, E)
    h = to_np(moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A)).copy()
    hf = orc.bf16_to_f32(h)
    assert np.all(np.isnan(hf[3])) and np.all(np.isnan(hf[7])) and not np.isnan(hf[[0, 1, 2, 4, 5, 6]]).any()
    h[[3, 7]] = 0
    coef = torch.full((M, A), 0.5, device=DEV)
    y = orc.bf16_to_f32(to_np(moe.experts_combine_grouped(torch.from_numpy(h.view(np.int16)).to(DEV).view(torch.bfloat16),
                                                          dn, E, tid, coef, ws, M, A)))
    assert np.all(np.isnan(y[1])) and np.all(np.isnan(y[3])) and not np.isnan(y[[0, 2]]).any()


def test_prefill_gemm_ragged_buckets_and_invalid_ids():
    """Prefill-size grouped GEMMs on skewed routing (buckets of 1 .. ~1000 slots, 128-slot pairs and lone 64-slot
    tiles) with invalid ids: valid rows match the F16-math model, invalid slots' rows are NaN."""
    say("prefill gemm ragged")
    M, A, E, H, I = 512, 4, 32, 256, 128
    gu, dn = _experts(4, E, H, I)
    x = orc.gen_bf16_normal(orc.tensor_key(6, "x"), 1.0, (M, H))
    rng = np.random.default_rng(11)
    p = 1.0 / np.arange(1, E + 1) ** 1.3
    ids = rng.choice(E, size=(M, A), p=p / p.sum()).astype(np.int32)
    ids[7, 1], ids[300, 3], ids[511, 0] = -1, E, E + 9
    tid = torch.from_numpy(ids).to(DEV)
    ws, err = moe.moe_group_routes(tid, E)
    h = to_np(moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A))
    b, q, s, m, G = qspec(gu)
    h16 = orc.experts_gate_up_swiglu_f16math(x, b, q, s, m, gu.N, H, G, E, ids)
    bad = np.array([7 * A + 1, 300 * A + 3, 511 * A + 0])
    good = np.setdiff1d(np.arange(M * A), bad)
    assert np.all(np.isnan(orc.bf16_to_f32(h[bad])))
    assert rel_err(h[good], h16[good]) < 2.0 ** -8
    hz = h.copy()
    hz[bad] = 0
    pt = torch.empty((M * A, H), dtype=torch.float32, device=DEV)
    coef = torch.full((M, A), 0.25, device=DEV)
    moe.experts_combine_grouped(torch.from_numpy(hz.view(np.int16)).to(DEV).view(torch.bfloat16), dn, E, tid, coef,
                                ws, M, A, partial=pt)
    b, q, s, m, G = qspec(dn)
    p16 = orc.experts_down_f16math(hz, b, q, s, m, dn.N, I, G, E, ids)
    # BF16 partials (ragged buckets, NT < 4 sub-tiles, invalid ids): the model rounded to BF16, NaN for invalid slots
    pb = _bf16_partials(pt)
    assert np.all(np.isnan(orc.bf16_to_f32(pb[bad])))
    assert rel_err(pb[good], orc.f32_to_bf16(p16[good])) <= 2.0 ** -8
    assert np.mean(pb[good] == orc.f32_to_bf16(p16[good])) > 0.99
    # the combine over BF16 partials: the ordered sum of the stored partials, NaN rows for the invalid ids' tokens
    y = moe.experts_combine_grouped(torch.from_numpy(hz.view(np.int16)).to(DEV).view(torch.bfloat16), dn, E, tid,
                                    coef, ws, M, A)
    yref, _ = orc.combine(orc.bf16_to_f32(pb), ids, np.full((M, A), 0.25, np.float32), E, H)
    yn = orc.bf16_to_f32(to_np(y))
    badtok = np.unique(bad // A)
    oktok = np.setdiff1d(np.arange(M), badtok)
    assert np.all(np.isnan(yn[badtok]))
    assert rel_err(to_np(y)[oktok], yref[oktok]) <= 2.0 ** -8


def test_perslot_kernels_match_grouped():
    say("per-slot")
    M, A, E, H, I = 3, 4, 16, 512, 128
    gu, dn = _experts(4, E, H, I)
    x = orc.gen_bf16_normal(orc.tensor_key(5, "x"), 1.0, (M, H))
    ids = np.random.default_rng(2).integers(0, E, (M, A)).astype(np.int32)
    tid = torch.from_numpy(ids).to(DEV)
    err = moe.zero_err()
    h = moe.experts_gather(bf16(x), gu, E, tid, err, swiglu=True)
    b, q, s, m, G = qspec(gu)
    href = orc.experts_gate_up_swiglu(x, orc.qview(b, q, s, m, gu.N, H, G), E, ids)
    assert rel_err(to_np(h), href) < 1e-2
    ws, _ = moe.moe_group_routes(tid, E)
    # the exact-weight kinds: the same per-slot MFMA sequence as the per-slot kernels, so the same bits
    ex = moe.MOE_MATH_WMMA_BF16
    hg = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A, math=ex)
    assert torch.equal(h, hg)
    g = moe.experts_gather(bf16(x), gu, E, tid, err)
    gg = moe.experts_gather_grouped(bf16(x), gu, E, ws, M, A, math=ex)
    assert torch.equal(g, gg)
    coef = torch.from_numpy(np.random.default_rng(3).random((M, A)).astype(np.float32)).to(DEV)
    y = moe.experts_combine(h, dn, E, tid, coef, err)
    yg = moe.experts_combine_grouped(h, dn, E, tid, coef, ws, M, A, math=ex)
    assert torch.equal(y, yg)  # per-slot dots summed over a in order: the same arithmetic
    assert to_np(err)[0] == 0
    bad = tid.clone()
    bad[1, 2] = E + 5
    y = moe.experts_combine(h, dn, E, bad, coef, err)
    assert torch.isnan(y[1].float()).all() and not torch.isnan(y[[0, 2]].float()).any()
    assert to_np(err).view(np.uint32).tolist() == [1, E + 5, 6]


@pytest.mark.parametrize("M,A,E", [(4, 6, 24), (40, 3, 6), (100, 10, 128)])
def test_decode_kernels_match_perslot(M, A, E):
    """The LDS-ring stream kernels at the served shape (H 3072, I 512, Q4 g128, the exact-weight kinds): h against the
    per-slot kernel, h and the down partials against the oracle. (4, 6, 24): the decode form (all M <= 16 tokens in the
    MFMA's rows); (40, 3, 6) puts 20 slots on each expert, so each expert has two token tiles, and (100, 10, 128)
    ~8: both take the gathered form (a tile's slots' rows), M above 16."""
    say("decode kernels vs per-slot", M, A, E)
    H, I = 3072, 512
    gu, dn = _experts(4, E, H, I, seed=13)
    x = orc.gen_bf16_normal(orc.tensor_key(6, "x"), 1.0, (M, H))
    ids = np.stack([np.random.default_rng(100 + m).permutation(E)[:A] for m in range(M)]).astype(np.int32)
    tid = torch.from_numpy(ids).to(DEV)
    err = moe.zero_err()
    ws, _ = moe.moe_group_routes(tid, E)
    ex = moe.MOE_MATH_WMMA_BF16  # the exact-weight kinds take the decode kernels
    hg = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A, math=ex)
    hp = moe.experts_gather(bf16(x), gu, E, tid, err, swiglu=True)
    # the decode gate_up splits K over a block's waves and adds their FP32 parts in K order; the per-slot kernel sums
    # over all of K in one wave: an h may round to the neighbouring bf16
    assert rel_err(to_np(hg), to_np(hp)) <= 2.0 ** -8
    assert (hg == hp).float().mean().item() > 0.95
    b, q, s, m, G = qspec(gu)
    href = orc.experts_gate_up_swiglu(x, orc.qview(b, q, s, m, gu.N, H, G), E, ids)
    assert rel_err(to_np(hg), href) < 1e-2
    coef = torch.from_numpy(np.random.default_rng(7).random((M, A)).astype(np.float32)).to(DEV)
    pt = torch.empty((M * A, H), dtype=torch.float32, device=DEV)
    yg = moe.experts_combine_grouped(hg, dn, E, tid, coef, ws, M, A, partial=pt, math=ex)
    b, q, s, m, G = qspec(dn)
    part = orc.experts_down(to_np(hg), orc.qview(b, q, s, m, dn.N, I, G), E, ids)
    assert rel_err(pt.cpu().numpy(), part) < 1e-4
    # the per-slot combine sums each group's activations on the VALU, the grouped kernels on the matrix cores: the
    # FP32 dots may differ in the last bits, so an output may round to the neighbouring bf16
    yp = moe.experts_combine(hg, dn, E, tid, coef, err)
    assert rel_err(to_np(yg), to_np(yp)) <= 2.0 ** -8
    assert to_np(err)[0] == 0


def test_linear_q8_and_swiglu():
    say("linear_q8 / swiglu")
    M, N, K = 20, 1024, 3072
    w = moe.QWeight.synth(8, 9, "sh_gu_q", "sh_gu_s", 0, N, K, 64)
    x = orc.gen_bf16_normal(orc.tensor_key(9, "x"), 1.0, (M, K))
    y = moe.linear_q8(bf16(x), w)
    spec = qspec(w)  # keep the host arrays alive while the view points at them
    ref = orc.dense(x, orc.qview(*spec[:4], N, K, 64))
    assert rel_err(to_np(y), ref) < 1e-2
    yf = moe.linear_q8(bf16(x), w, out_dtype=torch.float32)
    assert torch.equal(yf.to(torch.bfloat16), y)
    h = moe.swiglu(y, N // 2)
    href = orc.swiglu_bf16(to_np(y), N // 2)
    assert np.abs(to_np(h).astype(np.int32) - href.astype(np.int32)).max() <= 1  # expf ulps


@pytest.mark.parametrize("M,N,K", [(1, 1024, 3072), (16, 3072, 512), (37, 160, 1024), (300, 1024, 3072)])
def test_linear_q4_dense(M, N, K):
    """The dense Q4 projection (strixite kernels/linear_q4.hpp:23-31) against the oracle's dequantize-then-dot, FP32
    and BF16 outputs."""
    say("linear_q4", M, N, K)
    w = moe.QWeight.synth(4, 12, "gu_q", "gu_s", 3, N, K, 128)
    x = orc.gen_bf16_normal(orc.tensor_key(12, "x"), 1.0, (M, K))
    spec = qspec(w)
    ref = orc.dense(x, orc.qview(*spec[:4], N, K, 128))
    yf = moe.linear_q4(bf16(x), w, out_dtype=torch.float32)
    assert rel_err(yf.cpu().numpy(), ref) < 1e-5
    y = moe.linear_q4(bf16(x), w)
    assert torch.equal(yf.to(torch.bfloat16), y)


def test_shared_add_and_inject():
    say("shared add")
    M, N = 16, 3072
    rng = np.random.default_rng(4)
    y0 = orc.f32_to_bf16(rng.standard_normal((M, N)).astype(np.float32))
    s = orc.f32_to_bf16(rng.standard_normal((M, N)).astype(np.float32))
    gl = rng.standard_normal((M, 5)).astype(np.float32)
    gl[3, 2] = np.nan
    x = orc.f32_to_bf16(rng.standard_normal((M, 4 * N)).astype(np.float32))
    w_in = rng.standard_normal((M, 4)).astype(np.float32)
    y = bf16(y0.copy())
    err = moe.zero_err()
    moe.moe_shared_add(y, bf16(s), torch.from_numpy(np.ascontiguousarray(gl[:, 2])).to(DEV), 1, 512, err)
    g = 1 / (1 + np.exp(-gl[:, 2:3].astype(np.float64)))
    ref = orc.bf16_to_f32(y0) + g * orc.bf16_to_f32(s)
    got = orc.bf16_to_f32(to_np(y))
    assert np.all(np.isnan(got[3])) and to_np(err).view(np.uint32).tolist() == [1, 3, 512]
    ok = np.arange(M) != 3
    assert np.abs(got[ok] - ref[ok]).max() <= 2 ** -7 * np.abs(ref[ok]).max()
    # inject: bit-identical to the add then x += w_in * y on the stored y
    y2, xt, err2 = bf16(y0.copy()), bf16(x.copy()), moe.zero_err()
    glt = torch.from_numpy(gl).to(DEV)
    moe.moe_shared_add_inject(y2, bf16(s), glt[:, 1:], 5, 512, xt, torch.from_numpy(w_in).to(DEV), 4, err2)
    y3 = bf16(y0.copy())
    moe.moe_shared_add(y3, bf16(s), glt[:, 1:], 5, 512, moe.zero_err())
    assert torch.equal(y2, y3)
    xf = orc.bf16_to_f32(x).reshape(M, 4, N).astype(np.float64)
    xr = xf + w_in[:, :, None] * orc.bf16_to_f32(to_np(y3))[:, None, :]
    assert np.abs(orc.bf16_to_f32(to_np(xt)).reshape(M, 4, N) - xr).max() <= 2 ** -7 * np.abs(xr).max()


# ---- the sublayer ------------------------------------------------------------------------------------------------
def _layer_parity(layer, M, seed, logits_in=None, sample=None):
    x = moe.synth_bf16_normal(seed, "x", 0, (M, layer.H), 1.0)
    out = layer.forward(x, logits_in=logits_in)
    torch.cuda.synchronize()
    w = oracle_weights(layer)
    xn = to_np(x)
    rows = np.arange(M) if sample is None else np.sort(np.random.default_rng(seed).choice(M, sample, replace=False))
    lg = None if logits_in is None else np.ascontiguousarray(to_np(logits_in)[rows])
    o = orc.moe_layer(w, np.ascontiguousarray(xn[rows]), logits_in=lg)
    ids = to_np(out["ids"])
    assert np.array_equal(ids[rows], o["ids"]), "routing differs from the oracle"
    assert np.allclose(to_np(out["coef"])[rows], o["coef"], rtol=2e-6, atol=1e-7)
    e = rel_err(to_np(out["y"])[rows], o["y"])
    assert e < 1e-2, e
    assert rel_err(to_np(out["x_out"])[rows], o["out"]) < 1e-2
    assert to_np(out["err"])[0] == 0 and to_np(out["err"])[3] == 0
    if layer.shared_gate_up is not None:  # the routed experts made visible in y
        lb = balanced(layer)
        ob = lb.forward(x, logits_in=logits_in)
        torch.cuda.synchronize()
        rb = orc.moe_layer(oracle_weights(lb), np.ascontiguousarray(xn[rows]), logits_in=lg)
        assert np.array_equal(to_np(ob["ids"])[rows], rb["ids"])
        eb = rel_err(to_np(ob["y"])[rows], rb["y"])
        assert eb < 1e-2, ("balanced shared expert", eb)
    return out, o, e


@pytest.mark.parametrize("M,E,k", [(16, 64, 8), (128, 64, 8), (512, 512, 2), (3, 512, 10)])
def test_layer_fused_topk_packing_matches_router(M, E, k):
    """Small batches (M k <= 1024) route through one fused top-k + packing launch inside the layer: its ids and
    weights equal the standalone moe_router's bit for bit, ties and a non-finite token included, and the layer's
    output matches the same layer fed the standalone router's routing through the oracle's reference."""
    say("fused routing", M, E, k)
    layer = moe.MoeLayer.synth(256, E, k, 128, seed=3)
    rng = np.random.default_rng(M + E + k)
    ld = E + 1  # the layer's logits carry the shared-expert gate in column E
    lg = rng.standard_normal((M, ld)).astype(np.float32)
    lg[0, :E] = 0.5                      # all equal: ids 0..k-1
    if M > 2:
        lg[1, 2:2 + k + 2] = lg[1, :E].max() + 1  # a tie at the top
        lg[2, 5] = np.nan                 # a non-finite token
    x = moe.synth_bf16_normal(3, "x", 7, (M, 256), 1.0)
    out = layer.forward(x, logits_in=torch.from_numpy(lg).to(DEV))
    torch.cuda.synchronize()
    rids, rcoef, rerr = moe.moe_router(torch.from_numpy(np.ascontiguousarray(lg)).to(DEV), E, k, ld=ld)
    assert np.array_equal(to_np(out["ids"]), to_np(rids))
    assert np.array_equal(to_np(out["coef"]).view(np.uint32), to_np(rcoef).view(np.uint32))
    err = to_np(out["err"])
    if M > 2:
        assert err[0] == 1 and err[1] == 2 and err[2] == 5 and to_np(rerr)[0] == 1
        assert err[3] == 1, "the non-finite token's -1 ids reach the packing as invalid"
    else:
        assert err[0] == 0 and err[3] == 0
    # the routed part of the layer against the oracle on the finite tokens
    ok = np.all(np.isfinite(lg[:, :E]), axis=1)
    ws, _ = moe.moe_group_routes(rids, E)
    off, _, _ = orc.group_routes(to_np(rids), E)
    assert np.array_equal(to_np(moe.route_tables(ws, M, k, E)["offsets"]), off)
    assert np.all(np.isfinite(to_np(out["y"]).view(np.uint16)[ok] != 0x7fc0))


@pytest.mark.parametrize("M,H,biased", [(16, 3072, False), (5, 2048, True), (1, 4096, False)])
def test_layer_fused_router_launch(M, H, biased, monkeypatch):
    """Decode sizes with a shared expert can run the router projection, top-k and packing as one launch
    (STRIX_FUSED_ROUTE=1; the last router block to arrive routes): ids and coefficients equal linear_bf16w (+ bias) + moe_router bit for bit, y equals the
    same layer fed those logits (the separate top-k launch) bit for bit, on a workspace full of random bytes (the
    arrival ticket needs no clearing), on two calls in a row on it, and on three replays of a captured graph with
    other work between them (one epoch replayed: the last block's reset of the ticket)."""
    say("fused router launch", M, H, biased)
    E, k = 512, 10
    rng = np.random.default_rng(M + H)
    bias = torch.from_numpy((0.3 * rng.standard_normal(E)).astype(np.float32)).to(DEV) if biased else None
    layer = moe.MoeLayer.synth(H, E, k, 256, seed=9, router_bias=bias)
    x = moe.synth_bf16_normal(9, "x", M, (M, H), 1.0)
    lg = moe.linear_bf16w(x, layer.router)
    if biased:
        lg[:, :E] += bias
    rids, rcoef, _ = moe.moe_router(lg, E, k, ld=E + 1)
    want = layer.forward(x, logits_in=lg)
    torch.cuda.synchronize()
    monkeypatch.setenv("STRIX_FUSED_ROUTE", "1")
    ctx = moe.LayerContext()  # reads STRIX_FUSED_ROUTE once, at its creation

    def check(out, what):
        assert np.array_equal(to_np(out["ids"]), to_np(rids)), what
        assert np.array_equal(to_np(out["coef"]).view(np.uint32), to_np(rcoef).view(np.uint32)), what
        assert np.array_equal(to_np(out["y"]).view(np.uint16), to_np(want["y"]).view(np.uint16)), what
        assert to_np(out["err"])[0] == 0 and to_np(out["err"])[3] == 0, what

    ws = torch.from_numpy(rng.integers(0, 256, layer.workspace_bytes(M), dtype=np.uint8)).to(DEV)
    for call in range(2):
        out = layer.forward(x, ws=ws, ctx=ctx)
        torch.cuda.synchronize()
        check(out, ("call", call))
    # graph replays: the same launch arguments (epoch included) every replay
    out = {n: torch.zeros_like(t) for n, t in want.items()}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        layer.forward(x, ws=ws, out=out, ctx=ctx)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer.forward(x, ws=ws, out=out, ctx=ctx)
    for rep in range(3):
        for t in out.values():
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        check(out, ("replay", rep))
        layer.forward(x, ws=ws, ctx=ctx)  # eager work on the same workspace between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("biased", [False, True])
def test_layer_prefill_router_exact_routing(biased):
    """Prefill-size layers route through the bf16 MFMA projection + exact recomputation of the candidates: ids and
    coefficients equal the canonical-order router's (linear_bf16w + bias + moe_router) bit for bit, with exact ties
    (duplicated router rows), a block of all-zero rows, near ties one bf16 ulp apart, and a non-finite token, which
    takes the exact path for all its experts and raises the router error."""
    say("prefill router", biased)
    H, E, k, M = 1024, 64, 8, 512
    rng = np.random.default_rng(17)
    bias = torch.from_numpy((0.3 * rng.standard_normal(E)).astype(np.float32)).to(DEV) if biased else None
    layer = moe.MoeLayer.synth(H, E, k, 128, seed=5, router_bias=bias)
    r = layer.router
    rn = to_np(r).copy()
    rn[10:20] = rn[5]         # exact ties: equal logits, the lower index wins
    rn[30:40] = 0             # ten logits exactly 0
    rn[50] = rn[49]
    rn[50, 3] ^= 1            # one bf16 ulp apart in one element: near ties
    r.copy_(torch.from_numpy(rn.view(np.int16)).to(DEV).view(torch.bfloat16))
    x = moe.synth_bf16_normal(5, "x", 0, (M, H), 1.0)
    x[7, 100] = float("inf")  # a non-finite token
    x[9] = x[8]               # two identical tokens
    out = layer.forward(x)
    torch.cuda.synchronize()
    lg = moe.linear_bf16w(x, r)
    if biased:
        lg[:, :E] += bias  # one FP32 add, as the layer applies it
    rids, rcoef, rerr = moe.moe_router(lg, E, k, ld=E + 1)
    assert np.array_equal(to_np(out["ids"]), to_np(rids))
    assert np.array_equal(to_np(out["coef"]).view(np.uint32), to_np(rcoef).view(np.uint32))
    err = to_np(out["err"]).view(np.uint32)
    assert err[0] == 1 and err[1] == 7 and to_np(rerr).view(np.uint32)[0] == 1
    # and the canonical logits are the oracle's (the router itself is pinned there)
    ref = orc.router_logits(to_np(x), to_np(r), bias=to_np(bias) if biased else None)
    oids, _, _ = orc.topk(ref, E, k)
    ok = np.all(np.isfinite(ref[:, :E]), axis=1)
    assert np.array_equal(to_np(out["ids"])[ok], oids[ok])


def test_layer_config1_decode_q8():
    """1 token, H 2048, 64 experts, top-8, I 512, Q8 routed experts, no shared expert."""
    say("layer cfg1")
    layer = moe.MoeLayer.synth(2048, 64, 8, 512, seed=0, routed_bits=8, shared=False)
    _, _, e = _layer_parity(layer, 1, 0)
    say("cfg1 rel err", e)


def test_layer_config2_decode_16_tokens():
    """2 slots x (1 + 7 MTP drafts) = 16 tokens, H 3072, 512 experts, top-10 + shared Q8."""
    say("layer cfg2")
    layer = moe.MoeLayer.synth(3072, 512, 10, 512, seed=0)
    out, o, e = _layer_parity(layer, 16, 0)
    say("cfg2 rel err", e)
    # grouping of the layer's routing
    ws, _ = moe.moe_group_routes(out["ids"], 512)
    off, _, _ = orc.group_routes(o["ids"], 512)
    assert np.array_equal(to_np(moe.route_tables(ws, 16, 10, 512)["offsets"]), off)


def test_layer_config3_uniform_logits():
    """512-token prefill chunk with uniform random router logits (the router GEMV bypassed)."""
    say("layer cfg3")
    layer = moe.MoeLayer.synth(3072, 512, 10, 512, seed=0)
    lg = moe.synth_uniform_pm1(0, "logits", 0, (512, 513))
    out, _, _ = _layer_parity(layer, 512, 1, logits_in=lg)  # every token's output
    # routing on all 512 tokens: the top-k of the given logits
    rids, rcoef, _ = orc.topk(np.ascontiguousarray(to_np(lg)[:, :512]), 512, 10)
    assert np.array_equal(to_np(out["ids"]), rids)
    assert np.allclose(to_np(out["coef"]), rcoef, rtol=2e-6, atol=1e-7)


def test_layer_config4_zipf_prefill():
    """4096-token prefill, router biased to Zipf(1.1) expert popularity: every token's routing
    bit-exact and every token's output within tolerance (the oracle runs the whole layer on all 4096 tokens)."""
    say("layer cfg4")
    bias = torch.from_numpy(zipf_bias(0, 512, 1.0)).to(DEV)
    layer = moe.MoeLayer.synth(3072, 512, 10, 512, seed=0, router_bias=bias)
    out, o, e = _layer_parity(layer, 4096, 0)
    # routing on all tokens: the oracle's canonical logits for every token
    x = to_np(moe.synth_bf16_normal(0, "x", 0, (4096, 3072), 1.0))
    lg = orc.router_logits(x, to_np(layer.router), bias=to_np(bias))
    rids, _, _ = orc.topk(lg, 512, 10)
    assert np.array_equal(to_np(out["ids"]), rids)
    cnt = np.bincount(rids.ravel(), minlength=512)
    assert cnt.min() == 0 and cnt.max() > 400  # the load imbalance the config asks for


def test_layer_config5_stack_decode_then_prefill():
    """BASELINE config 5 as the bench runs it: a stack of 8 consecutive layers with independent per-layer weights and
    Zipf router biases drawn from the seed, a 16-token decode step and then a 4096-token prefill step back to back,
    captured as ONE HIP graph (one workspace a step, the buffers of every layer live). The graph is replayed twice
    with every output poisoned in between (a fill kernel, so the checked values come from the second replay). Each
    layer takes its own seeded input, as the bench does (the sublayer has no normalization, so feeding x_out on
    unnormalized synthetic weights would grow without bound). Every layer of both steps: ids bit-exact on every token,
    y and x_out on sampled tokens against the oracle, no error words (the reference's per-layer order,
    strixite runtime/qwen4exp.cpp:3143-3217)."""
    say("layer cfg5")
    NL, H, E, k, I = 8, 3072, 512, 10, 512
    layers = []
    for l in range(NL):
        bias = torch.from_numpy(zipf_bias(l, E, 1.0)).to(DEV)
        layers.append(moe.MoeLayer.synth(H, E, k, I, seed=0, layer=l, router_bias=bias))
    ctx = moe.LayerContext()
    steps = {}
    for M in (16, 4096):
        ws = layers[0].workspace(M)
        ins = [moe.synth_bf16_normal(5, "x", 100 * M + l, (M, H), 1.0) for l in range(NL)]
        outs = [layers[l].forward(ins[l], ws=ws, ctx=ctx) for l in range(NL)]  # eager: allocates the outputs
        steps[M] = (ins, outs, ws)
    torch.cuda.synchronize()

    def stack():
        for M in (16, 4096):
            ins, outs, ws = steps[M]
            for l in range(NL):
                layers[l].forward(ins[l], ws=ws, out=outs[l], ctx=ctx)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        stack()
    torch.cuda.synchronize()
    say("cfg5 captured")
    for rep in range(2):
        for M in (16, 4096):
            for o in steps[M][1]:
                o["ids"].fill_(-7)
                o["coef"].fill_(float("nan"))
                o["y"].fill_(float("nan"))
                o["x_out"].fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        say("cfg5 replay", rep)
    for M in (16, 4096):
        ins, outs, _ = steps[M]
        for l in range(NL):
            say("cfg5 check", M, l)
            w = oracle_weights(layers[l])
            xn = to_np(ins[l])
            lg = orc.router_logits(xn, w["router"], bias=w["router_bias"])
            rids, _, _ = orc.topk(lg, E, k)
            assert np.array_equal(to_np(outs[l]["ids"]), rids), (M, l)
            rows = np.arange(M) if M <= 16 else np.sort(np.random.default_rng(l).choice(M, 32, replace=False))
            o = orc.moe_layer(w, np.ascontiguousarray(xn[rows]))
            assert np.array_equal(to_np(outs[l]["ids"])[rows], o["ids"])
            assert rel_err(to_np(outs[l]["y"])[rows], o["y"]) < 1e-2, (M, l)
            assert rel_err(to_np(outs[l]["x_out"])[rows], o["out"]) < 1e-2, (M, l)
            assert to_np(outs[l]["err"])[0] == 0 and to_np(outs[l]["err"])[3] == 0
    del g
    # the routed experts made visible in y: the first layer again, balanced, at both sizes
    for M in (16, 4096):
        lb = balanced(layers[0])
        x = steps[M][0][0]
        ob = lb.forward(x, ctx=ctx)
        torch.cuda.synchronize()
        rows = np.arange(M) if M <= 16 else np.sort(np.random.default_rng(7).choice(M, 32, replace=False))
        rb = orc.moe_layer(oracle_weights(lb), np.ascontiguousarray(to_np(x)[rows]))
        assert np.array_equal(to_np(ob["ids"])[rows], rb["ids"])
        assert rel_err(to_np(ob["y"])[rows], rb["y"]) < 1e-2, ("balanced", M)


@pytest.mark.parametrize("M", [16, 600])
def test_layer_hyperconnection_inject(M):
    """The layer's residual end with hyper-connections (strixite runtime/qwen4exp.cpp:3206-3216): the stored y injected
    into 4 residual streams in place by the combine's epilogue equals the layer without it followed by the standalone
    hc_inject bit for bit, and hc_inject equals its closed form xs + w_in * y (one FP32 fma, one bf16 rounding)."""
    say("hc inject", M)
    layer = moe.MoeLayer.synth(1024, 64, 8, 256, seed=8)
    x = moe.synth_bf16_normal(8, "x", 1, (M, 1024), 1.0)
    rng = np.random.default_rng(M)
    xs0 = orc.f32_to_bf16(rng.standard_normal((M, 4 * 1024)).astype(np.float32))
    w_in = torch.from_numpy((2 / (1 + np.exp(-rng.standard_normal((M, 4))))).astype(np.float32)).to(DEV)
    xs = bf16(xs0.copy())
    out = layer.forward(x, inject=(xs, w_in))
    ref = layer.forward(x)
    xr = bf16(xs0.copy())
    moe.hc_inject(xr, w_in, ref["y"])
    torch.cuda.synchronize()
    assert torch.equal(out["y"], ref["y"]) and torch.equal(out["ids"], ref["ids"])
    assert torch.equal(xs, xr)
    # closed form: fma in float64 (exact product), rounded to FP32, then to bf16
    yv = orc.bf16_to_f32(to_np(ref["y"])).astype(np.float64)
    wv = to_np(w_in).astype(np.float64)
    cf = (wv[:, :, None] * yv[:, None, :] + orc.bf16_to_f32(xs0).reshape(M, 4, 1024)).astype(np.float32)
    want = orc.f32_to_bf16(cf.reshape(M, 4 * 1024))
    got = to_np(xs)
    assert np.mean(got == want) > 0.9999 and np.abs(got.astype(np.int32) - want.astype(np.int32)).max() <= 1


@pytest.mark.parametrize("M", [16, 120, 512])
def test_layer_stacked_shared_expert(M):
    """The converter's default layout (strixite formats/merge_plan.cpp:31-41): the shared expert is expert E of the
    stacked routed tensors, routed as slot k of every token with coefficient sigmoid(router row E) (strixite
    kernels/moe_router.hip:108-111). Decode-size (one-launch top-k + packing), mid-size (moe_router) and prefill-size
    (the MFMA router) batches: ids and coefficients against the oracle, every token; output on seeded tokens."""
    say("stacked shared", M)
    H, E, k, I = 1024, 64, 8, 256
    layer = moe.MoeLayer.synth(H, E, k, I, seed=9, shared="stacked")
    x = moe.synth_bf16_normal(9, "x", M, (M, H), 1.0)
    out = layer.forward(x)
    torch.cuda.synchronize()
    w = oracle_weights(layer)
    xn = to_np(x)
    rows = np.arange(M) if M <= 16 else np.sort(np.random.default_rng(M).choice(M, 24, replace=False))
    o = orc.moe_layer(w, np.ascontiguousarray(xn[rows]))
    ids = to_np(out["ids"])
    assert ids.shape == (M, k + 1) and np.all(ids[:, k] == E)
    lg = orc.router_logits(xn, w["router"])
    rids, rcoef, _ = orc.topk(lg, E, k, shared=np.ascontiguousarray(lg[:, E:]), shared_ld=1, shared_id=E)
    assert np.array_equal(ids, rids)
    assert np.allclose(to_np(out["coef"]), rcoef, rtol=2e-6, atol=1e-7)
    assert np.array_equal(ids[rows], o["ids"])
    assert rel_err(to_np(out["y"])[rows], o["y"]) < 1e-2
    assert rel_err(to_np(out["x_out"])[rows], o["out"]) < 1e-2
    assert to_np(out["err"])[0] == 0 and to_np(out["err"])[3] == 0


def test_layer_stacked_shared_nonfinite_gate():
    """A non-finite shared-expert gate logit marks the token as the reference's router does: every slot -1, its
    coefficients NaN, the router error naming expert E; the other tokens route normally."""
    say("stacked shared nonfinite")
    H, E, k, I, M = 1024, 64, 8, 256, 6
    layer = moe.MoeLayer.synth(H, E, k, I, seed=10, shared="stacked")
    lg = np.random.default_rng(2).standard_normal((M, E + 1)).astype(np.float32)
    lg[3, E] = np.inf
    x = moe.synth_bf16_normal(10, "x", 0, (M, H), 1.0)
    out = layer.forward(x, logits_in=torch.from_numpy(lg).to(DEV))
    torch.cuda.synchronize()
    ids = to_np(out["ids"])
    assert np.all(ids[3] == -1) and np.all(np.isnan(to_np(out["coef"])[3]))
    e = to_np(out["err"]).view(np.uint32)
    assert e[0] == 1 and e[1] == 3 and e[2] == E
    rids, _, _ = orc.topk(lg, E, k, shared=np.ascontiguousarray(lg[:, E:]), shared_ld=1, shared_id=E)
    assert np.array_equal(ids, rids)
    ok = np.arange(M) != 3
    assert not np.isnan(orc.bf16_to_f32(to_np(out["y"])[ok])).any()


# ---- quantization groups below the 16-byte K step (Q4 G 64 / 32, Q8 G 32) ----------------------------------------
@pytest.mark.parametrize("bits,G,M,A,E,H,I", [(4, 64, 16, 10, 64, 512, 256), (4, 32, 16, 10, 64, 512, 256),
                                              (8, 32, 5, 8, 32, 512, 128), (4, 64, 300, 8, 16, 256, 128),
                                              (4, 32, 300, 8, 16, 256, 128)])
def test_grouped_small_groups(bits, G, M, A, E, H, I):
    """G = 64 is the converter's default Q4 layout (strixite formats/convert_qwen4exp.hpp:37, default=q4g64). With G
    below the load's span the K step is one group; decode (M 16: the stream kernels) and prefill sizes (M 300: the
    exact-weight GEMM at G 64, the stream kernels at G 32) under the exact kinds: h and the FP32 down partials against
    the oracle; Q4 under the F16 kinds (a group a chunk at G 64, a group a lane half at G 32): h and the BF16 partials
    against the F16 math's model."""
    say("small groups", bits, G, M, A, E, H, I)
    gu = moe.QWeight.synth(bits, 17, "gu_q", "gu_s", 0, E * 2 * I, H, G)
    dn = moe.QWeight.synth(bits, 17, "dn_q", "dn_s", 0, E * H, I, G)
    x = orc.gen_bf16_normal(orc.tensor_key(17, "x"), 1.0, (M, H))
    ids = np.stack([np.random.default_rng(300 + m).permutation(E)[:A] for m in range(M)]).astype(np.int32)
    tid = torch.from_numpy(ids).to(DEV)
    ws, _ = moe.moe_group_routes(tid, E)
    ex = moe.MOE_MATH_WMMA_BF16
    h = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A, math=ex)
    b, q, s, m, G_ = qspec(gu)
    href = orc.experts_gate_up_swiglu(x, orc.qview(b, q, s, m, gu.N, H, G_), E, ids)
    assert G_ == G and rel_err(to_np(h), href) < 1e-2
    if bits == 4:
        h16 = moe.experts_gather_grouped_swiglu(bf16(x), gu, E, ws, M, A)
        m16 = orc.experts_gate_up_swiglu_f16math(x, b, q, s, m, gu.N, H, G, E, ids)
        assert rel_err(to_np(h16), m16) < 2.0 ** -8
    coef = torch.from_numpy(np.random.default_rng(6).random((M, A)).astype(np.float32)).to(DEV)
    if bits == 4:
        p16 = torch.empty((M * A, H), dtype=torch.float32, device=DEV)
        moe.experts_combine_grouped(h, dn, E, tid, coef, ws, M, A, partial=p16)
        bd, qd, sd, md, _ = qspec(dn)
        pm = orc.f32_to_bf16(orc.experts_down_f16math(to_np(h), bd, qd, sd, md, dn.N, I, G, E, ids))
        pb = _bf16_partials(p16)
        assert rel_err(pb, pm) <= 2.0 ** -8 and np.mean(pb == pm) > 0.99
    pt = torch.empty((M * A, H), dtype=torch.float32, device=DEV)
    y = moe.experts_combine_grouped(h, dn, E, tid, coef, ws, M, A, partial=pt, math=ex)
    b, q, s, m, _ = qspec(dn)
    part = orc.experts_down(to_np(h), orc.qview(b, q, s, m, dn.N, I, G), E, ids)
    assert rel_err(pt.cpu().numpy(), part) < 1e-4
    yref, _ = orc.combine(part, ids, to_np(coef), E, H)
    assert rel_err(to_np(y), yref) < 1e-2
    if bits == 4 and M <= 16:  # the per-slot kernels: the same per-slot MFMA sequence as the grouped ones
        err = moe.zero_err()
        hp = moe.experts_gather(bf16(x), gu, E, tid, err, swiglu=True)
        assert torch.equal(hp, h)
        yp = moe.experts_combine(h, dn, E, tid, coef, err)
        assert rel_err(to_np(yp), to_np(y)) <= 2.0 ** -8
        assert to_np(err)[0] == 0


@pytest.mark.parametrize("bits,G,M", [(4, 64, 7), (4, 32, 7), (8, 32, 7), (4, 64, 200), (8, 64, 200), (8, 32, 200)])
def test_dense_small_groups(bits, G, M):
    """Decode sizes on the stream kernels, prefill sizes (M >= 128) on the matrix-core GEMM (G 64 / 128) or the stream
    kernels (G 32)."""
    say("dense small groups", bits, G, M)
    N, K = 320, 1024
    w = moe.QWeight.synth(bits, 18, "gu_q", "gu_s", 1, N, K, G)
    x = orc.gen_bf16_normal(orc.tensor_key(18, "x"), 1.0, (M, K))
    spec = qspec(w)
    ref = orc.dense(x, orc.qview(*spec[:4], N, K, G))
    f = moe.linear_q4 if bits == 4 else moe.linear_q8
    yf = f(bf16(x), w, out_dtype=torch.float32)
    assert rel_err(yf.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("G,shared_G,M", [(64, 64, 16), (64, 64, 600), (32, 32, 16), (32, 64, 200)])
def test_layer_small_groups(G, shared_G, M):
    """The whole sublayer with Q4 G 64 / 32 routed experts (a Q8 G 32 shared expert runs beside the routed launches
    rather than riding along): routing bit-exact, output within 1e-2 of the oracle on seeded rows."""
    say("layer small groups", G, shared_G, M)
    H, E, k, I = 1024, 64, 8, 256
    layer = moe.MoeLayer.synth(H, E, k, I, seed=21, routed_G=G, shared_G=shared_G)
    x = moe.synth_bf16_normal(21, "x", M, (M, H), 1.0)
    out = layer.forward(x)
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 16 else np.sort(np.random.default_rng(M).choice(M, 24, replace=False))
    o = orc.moe_layer(oracle_weights(layer), np.ascontiguousarray(to_np(x)[rows]))
    assert np.array_equal(to_np(out["ids"])[rows], o["ids"])
    assert rel_err(to_np(out["y"])[rows], o["y"]) < 1e-2
    assert not to_np(out["err"]).any()


@pytest.mark.parametrize("G,H,I,M", [(128, 384, 256, 600), (64, 320, 192, 600), (128, 640, 128, 300)])
def test_layer_partial_spans(G, H, I, M):
    """The prefill GEMMs' K loop at sizes where K is not a whole number of 4-chunk code spans (K = 320, 384, 640,
    192 ...) and G 128 groups come in odd numbers a row (the scales then load a group at a time): routing bit-exact,
    output within 1e-2 of the oracle on seeded rows."""
    say("layer partial spans", G, H, I, M)
    E, k = 64, 8
    layer = moe.MoeLayer.synth(H, E, k, I, seed=23, routed_G=G, shared_G=64)
    x = moe.synth_bf16_normal(23, "x", M, (M, H), 1.0)
    out = layer.forward(x)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(M).choice(M, 24, replace=False))
    o = orc.moe_layer(oracle_weights(layer), np.ascontiguousarray(to_np(x)[rows]))
    assert np.array_equal(to_np(out["ids"])[rows], o["ids"])
    assert rel_err(to_np(out["y"])[rows], o["y"]) < 1e-2
    assert not to_np(out["err"]).any()
