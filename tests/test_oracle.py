"""Pins the CPU oracle (oracle/) before anything is checked against it: golden vectors from the reference's own
quantizers, closed forms, brute force on tiny inputs and invariants -- chosen so that a dropped term, a wrong
index or a transposed operand fails one of them."""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "formats.npz")


# ---- bf16 -----------------------------------------------------------------------------------------------------
def test_bf16_known_answers(orc):
    L = orc.lib()
    assert L.orc_f32_to_bf16(1.0) == 0x3F80
    assert L.orc_f32_to_bf16(-2.0) == 0xC000
    # halfway cases round to even: 1 + 2^-8 -> 1.0 (even), 1 + 3*2^-8 -> 1 + 2^-6 (even mantissa)
    assert L.orc_f32_to_bf16(1.0 + 2.0 ** -8) == 0x3F80
    assert L.orc_f32_to_bf16(1.0 + 3 * 2.0 ** -8) == 0x3F82
    assert L.orc_f32_to_bf16(float("inf")) == 0x7F80
    assert L.orc_f32_to_bf16(float("nan")) & 0x7FC0 == 0x7FC0
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32)
    b = orc.f32_to_bf16(x)
    # RNE: the result is one of the two neighbours and the nearer one
    back = orc.bf16_to_f32(b).astype(np.float64)
    up = orc.bf16_to_f32(b + 1).astype(np.float64)
    dn = orc.bf16_to_f32(b - 1).astype(np.float64)
    err = np.abs(back - x)
    assert np.all(err <= np.abs(up - x)) and np.all(err <= np.abs(dn - x))
    assert all(L.orc_f32_to_bf16(float(v)) == int(bb) for v, bb in zip(x[:200], b[:200]))


# ---- formats: the reference's own quantizer output ------------------------------------------------------------
@pytest.mark.parametrize("name", ["normal", "edge", "halfway", "wide"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_formats_match_reference_golden(orc, name, bits, G):
    g = np.load(GOLDEN)
    tag = f"{name}_q{bits}_g{G}"
    w = g[tag + "_w"]
    N, K = w.shape
    q, s, m = orc.quantize(bits, w, G)
    assert np.array_equal(q, g[tag + "_q"]) and np.array_equal(s, g[tag + "_s"]) and np.array_equal(m, g[tag + "_m"])
    d = orc.dequantize(bits, g[tag + "_q"], g[tag + "_s"], g[tag + "_m"], N, K, G)
    assert np.array_equal(d.view(np.uint32), g[tag + "_deq"].view(np.uint32))


def test_formats_refusals_match_reference(orc):
    g = np.load(GOLDEN)
    with pytest.raises(ValueError):
        orc.quantize(4, np.array([[1.0, np.nan] * 16], np.float32), 32)
    assert bool(g["refuses_nan"])
    with pytest.raises(ValueError):
        orc.quantize(4, np.ones((1, 32), np.float32), 16)
    assert bool(g["refuses_g16"])


def test_dequant_closed_form(orc):
    # code 0 -> m, code 15 -> 15 s + m, low nibble = even k (formats/q4.hpp:3-6)
    s_b, m_b = orc.f32_to_bf16(np.array([0.5], np.float32)), orc.f32_to_bf16(np.array([-3.0], np.float32))
    q = np.zeros(16, np.uint8)
    q[0] = 0xF0  # k=0 -> 0, k=1 -> 15
    d = orc.dequantize(4, q, s_b, m_b, 1, 32, 32)
    assert d[0, 0] == -3.0 and d[0, 1] == 15 * 0.5 - 3.0 and np.all(d[0, 2:] == -3.0)
    q8 = np.zeros(32, np.uint8)
    q8[3] = 255
    d8 = orc.dequantize(8, q8, s_b, m_b, 1, 32, 32)
    assert d8[0, 3] == np.float32(255 * 0.5) - 3.0 and d8[0, 0] == -3.0


# ---- generator ------------------------------------------------------------------------------------------------
def test_generator_statistics_and_layout(orc):
    key = orc.tensor_key(0, "x")
    x = orc.bf16_to_f32(orc.gen_bf16_normal(key, 1.0, 200000))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01 and np.abs(x).max() <= 3.47
    assert np.array_equal(orc.gen_bf16_normal(key, 1.0, 1000), orc.gen_bf16_normal(key, 1.0, 1000))
    q, s, m = orc.gen_q(4, orc.tensor_key(0, "gu_q"), orc.tensor_key(0, "gu_s"), 64, 256, 128)
    sf, mf = orc.bf16_to_f32(s), orc.bf16_to_f32(m)
    assert np.all(mf == -8 * sf) and np.all(sf >= 0)  # w = (u - 8) s exactly
    codes = np.stack([q & 15, q >> 4], 1).ravel()
    assert np.bincount(codes, minlength=16).min() > 0.8 * codes.size / 16
    q8, s8, m8 = orc.gen_q(8, orc.tensor_key(0, "sh_gu_q"), orc.tensor_key(0, "sh_gu_s"), 16, 256, 64)
    assert q8.min() >= 1 and np.all(orc.bf16_to_f32(m8) == -128 * orc.bf16_to_f32(s8))
    u = orc.gen_uniform_pm1(orc.tensor_key(0, "logits"), 100000)
    assert u.min() >= -1.0 and u.max() < 1.0 and abs(u.mean()) < 0.01


# ---- router logits: the canonical order ------------------------------------------------------------------------
def _canonical_numpy(x, w):
    """Independent restatement: bf16 x bf16 products are exact in f32, so fmaf(x, w, acc) == f32(acc + x*w)."""
    xf, wf = x.astype(np.float32), w.astype(np.float32)
    K = xf.shape[-1]
    chunks = (K + 7) // 8
    lanes = np.zeros(64, np.float32)
    for l in range(64):
        acc = np.float32(0)
        for c in range(l, chunks, 64):
            for i in range(8):
                k = c * 8 + i
                if k < K:
                    acc = np.float32(acc + np.float32(xf[k] * wf[k]))
        lanes[l] = acc
    off = 32
    while off:
        lanes[:off] = lanes[:off] + lanes[off:2 * off]
        off //= 2
    return lanes[0]


@pytest.mark.parametrize("K", [512, 1000, 3072])
def test_router_logits_canonical_order(orc, K):
    rng = np.random.default_rng(K)
    x = orc.f32_to_bf16(rng.standard_normal((3, K)).astype(np.float32))
    w = orc.f32_to_bf16((rng.standard_normal((5, K)) * 0.02).astype(np.float32))
    y = orc.router_logits(x, w)
    xf, wf = orc.bf16_to_f32(x), orc.bf16_to_f32(w)
    for m in range(3):
        for n in range(5):
            assert y[m, n] == _canonical_numpy(xf[m], wf[n])
    exact = xf.astype(np.float64) @ wf.astype(np.float64).T
    bound = 64 * K * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(y - exact) <= bound)
    bias = rng.standard_normal(4).astype(np.float32)
    yb = orc.router_logits(x, w, bias)
    assert np.array_equal(yb[:, :4], y[:, :4] + bias) and np.array_equal(yb[:, 4], y[:, 4])


# ---- top-k -----------------------------------------------------------------------------------------------------
def _topk_brute(row, k):
    order = sorted(range(len(row)), key=lambda e: (-row[e], e))
    return order[:k]


@pytest.mark.parametrize("E,k", [(8, 3), (64, 8), (512, 10), (1024, 32), (7, 7)])
def test_topk_brute_force(orc, E, k):
    rng = np.random.default_rng(E + k)
    lg = rng.standard_normal((20, E)).astype(np.float32)
    lg[3, :] = 0.5  # all equal -> ids 0..k-1
    lg[4, 5:9] = lg[4].max() + 1  # a four-way tie at the top
    ids, coef, err = orc.topk(lg, E, k)
    assert err[0] == 0
    for m in range(20):
        assert list(ids[m]) == _topk_brute(lg[m], k)
        v = lg[m, ids[m]].astype(np.float64)
        p = np.exp(v - v.max())
        assert np.allclose(coef[m], p / p.sum(), rtol=2e-6, atol=1e-7)
        assert abs(coef[m].sum() - 1) < 1e-5
    assert list(ids[3]) == list(range(k))


def test_topk_shared_and_nonfinite(orc):
    E, k = 16, 4
    lg = np.random.default_rng(1).standard_normal((6, E + 1)).astype(np.float32)
    lg[2, 7] = np.nan
    lg[4, 3] = -np.inf
    lg[5, E] = np.inf  # the shared gate
    ids, coef, err = orc.topk(lg, E, k, shared=lg[:, E:].copy(), shared_ld=1, shared_id=E)
    assert list(err) == [1, 2, 7]  # first failing token in token order, its smallest bad expert
    for m in (2, 4, 5):
        assert np.all(ids[m] == -1) and np.all(np.isnan(coef[m]))
    for m in (0, 1, 3):
        assert ids[m, k] == E and abs(coef[m, k] - 1 / (1 + np.exp(-lg[m, E]))) < 1e-6
        assert list(ids[m, :k]) == _topk_brute(lg[m, :E], k)


# ---- packing ---------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,A,E", [(1, 8, 64), (16, 10, 512), (300, 10, 512), (7, 3, 5)])
def test_group_routes_counting_sort(orc, M, A, E):
    rng = np.random.default_rng(M * A)
    ids = rng.integers(0, E, (M, A)).astype(np.int32)
    if M > 5:
        ids[2, 1] = -1
        ids[5, 0] = E
    offsets, slots, err = orc.group_routes(ids, E)
    flat = ids.ravel()
    bucket = np.where((flat < 0) | (flat >= E), E, flat)
    cnt = np.bincount(bucket, minlength=E + 1)
    assert np.array_equal(offsets[:-1], np.concatenate([[0], np.cumsum(cnt)[:-1]]))
    assert offsets[-1] == M * A
    assert np.array_equal(slots, np.argsort(bucket, kind="stable"))
    if M > 5:
        assert list(err) == [1, 0xFFFFFFFF, 2 * A + 1]
    else:
        assert err[0] == 0


# ---- expert math -----------------------------------------------------------------------------------------------
def _tiny_layer(orc, M=5, H=256, E=4, k=2, I=128, bits=4, G=128, shared=True, seed=3):
    key = lambda t: orc.tensor_key(seed, t)  # noqa: E731
    w = {"E": E, "k": k, "I": I}
    w["router"] = orc.gen_bf16_normal(key("router"), 0.02, (E + (1 if shared else 0), H))
    gsh = 64 if G == 128 else G
    w["gu"] = (bits, *orc.gen_q(bits, key("gu_q"), key("gu_s"), E * 2 * I, H, G), G)
    w["dn"] = (bits, *orc.gen_q(bits, key("dn_q"), key("dn_s"), E * H, I, G), G)
    if shared:
        w["sh_gu"] = (8, *orc.gen_q(8, key("sh_gu_q"), key("sh_gu_s"), 2 * I, H, gsh), gsh)
        w["sh_dn"] = (8, *orc.gen_q(8, key("sh_dn_q"), key("sh_dn_s"), H, I, gsh), gsh)
    x = orc.gen_bf16_normal(key("x"), 1.0, (M, H))
    return w, x


def _deq(orc, spec, N, K):
    bits, q, s, m, G = spec
    return orc.dequantize(bits, q, s, m, N, K, G).astype(np.float64)


def _silu(v):
    return v / (1 + np.exp(-v))


def test_layer_closed_form(orc):
    """y = sum_a coef * Wd[id] (silu(Wg[id] x) * Wu[id] x) + sigmoid(g) shared(x), in float64 from dequantized
    weights, against the oracle's FP32 layer (rounding points bf16)."""
    w, x = _tiny_layer(orc)
    E, k, I = w["E"], w["k"], w["I"]
    M, H = x.shape
    o = orc.moe_layer(w, x)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    gu, dn = _deq(orc, w["gu"], E * 2 * I, H), _deq(orc, w["dn"], E * H, I)
    shgu, shdn = _deq(orc, w["sh_gu"], 2 * I, H), _deq(orc, w["sh_dn"], H, I)
    lg = xf @ orc.bf16_to_f32(w["router"]).astype(np.float64).T
    assert np.allclose(o["logits"], lg, rtol=1e-5, atol=1e-5)
    for m in range(M):
        assert list(o["ids"][m]) == _topk_brute(o["logits"][m, :E], k)
    y = np.zeros((M, H))
    for m in range(M):
        for a in range(k):
            e = o["ids"][m, a]
            g = gu[e * 2 * I:e * 2 * I + I] @ xf[m]
            u = gu[e * 2 * I + I:(e + 1) * 2 * I] @ xf[m]
            h = _silu(g) * u
            y[m] += o["coef"][m, a] * (dn[e * H:(e + 1) * H] @ h)
        g = shgu[:I] @ xf[m]
        u = shgu[I:] @ xf[m]
        y[m] += 1 / (1 + np.exp(-lg[m, E])) * (shdn @ (_silu(g) * u))
    got = orc.bf16_to_f32(o["y"]).astype(np.float64)
    assert np.abs(got - y).max() / np.abs(y).max() < 1e-2
    out = orc.bf16_to_f32(o["out"]).astype(np.float64)
    assert np.abs(out - (xf + got)).max() <= np.abs(xf + got).max() * 2 ** -8


def test_layer_stacked_shared_closed_form(orc):
    """Shared expert stacked as expert E of the routed tensors and routed as slot k: the same float64 sum, with the
    shared term taken from rows E of gate_up / down and the id / coefficient of slot k checked as E / sigmoid(g)."""
    E, k, I, H, M, seed = 4, 2, 128, 256, 5, 4
    key = lambda t: orc.tensor_key(seed, t)  # noqa: E731
    w = {"E": E, "k": k, "I": I, "shared_stacked": True}
    w["router"] = orc.gen_bf16_normal(key("router"), 0.02, (E + 1, H))
    w["gu"] = (4, *orc.gen_q(4, key("gu_q"), key("gu_s"), (E + 1) * 2 * I, H, 128), 128)
    w["dn"] = (4, *orc.gen_q(4, key("dn_q"), key("dn_s"), (E + 1) * H, I, 128), 128)
    x = orc.gen_bf16_normal(key("x"), 1.0, (M, H))
    o = orc.moe_layer(w, x)
    assert o["ids"].shape == (M, k + 1) and np.all(o["ids"][:, k] == E)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    gu, dn = _deq(orc, w["gu"], (E + 1) * 2 * I, H), _deq(orc, w["dn"], (E + 1) * H, I)
    lg = xf @ orc.bf16_to_f32(w["router"]).astype(np.float64).T
    assert np.allclose(o["coef"][:, k], 1 / (1 + np.exp(-lg[:, E])), rtol=1e-5)
    y = np.zeros((M, H))
    for m in range(M):
        assert list(o["ids"][m, :k]) == _topk_brute(o["logits"][m, :E], k)
        for a in range(k + 1):
            e = o["ids"][m, a]
            g = gu[e * 2 * I:e * 2 * I + I] @ xf[m]
            u = gu[e * 2 * I + I:(e + 1) * 2 * I] @ xf[m]
            y[m] += o["coef"][m, a] * (dn[e * H:(e + 1) * H] @ (_silu(g) * u))
    got = orc.bf16_to_f32(o["y"]).astype(np.float64)
    assert np.abs(got - y).max() / np.abs(y).max() < 1e-2
    # dropping the shared term must be visible at this tolerance
    ysh = np.zeros((M, H))
    for m in range(M):
        g = gu[E * 2 * I:E * 2 * I + I] @ xf[m]
        u = gu[E * 2 * I + I:(E + 1) * 2 * I] @ xf[m]
        ysh[m] = o["coef"][m, k] * (dn[E * H:(E + 1) * H] @ (_silu(g) * u))
    assert np.abs(ysh).max() / np.abs(y).max() > 5e-2


def test_experts_down_and_dense(orc):
    w, x = _tiny_layer(orc, shared=True, M=3)
    E, I = w["E"], w["I"]
    H = x.shape[1]
    ids = np.array([[0, 3], [2, 2], [1, 0]], np.int32)
    bits, q, s, m, G = w["gu"]
    h = orc.experts_gate_up_swiglu(x, orc.qview(bits, q, s, m, E * 2 * I, H, G), E, ids)
    gu = _deq(orc, w["gu"], E * 2 * I, H)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    for mm in range(3):
        for a in range(2):
            e = ids[mm, a]
            ref = _silu(gu[e * 2 * I:e * 2 * I + I] @ xf[mm]) * (gu[e * 2 * I + I:(e + 1) * 2 * I] @ xf[mm])
            got = orc.bf16_to_f32(h[mm * 2 + a])
            assert np.abs(got - ref).max() <= np.abs(ref).max() * 2 ** -7
    bits, q, s, m, G = w["dn"]
    p = orc.experts_down(h, orc.qview(bits, q, s, m, E * H, I, G), E, ids)
    dn = _deq(orc, w["dn"], E * H, I)
    hf = orc.bf16_to_f32(h).astype(np.float64)
    for sl in range(6):
        e = ids.ravel()[sl]
        assert np.allclose(p[sl], dn[e * H:(e + 1) * H] @ hf[sl], rtol=1e-4, atol=1e-4)
    bits, q, s, m, G = w["sh_gu"]
    d = orc.dense(x, orc.qview(bits, q, s, m, 2 * I, H, G))
    assert np.allclose(d, xf @ _deq(orc, w["sh_gu"], 2 * I, H).T, rtol=1e-4, atol=1e-4)


def test_combine_order_and_invalid(orc):
    rng = np.random.default_rng(5)
    M, A, E, N = 3, 4, 8, 16
    ids = rng.integers(0, E, (M, A)).astype(np.int32)
    ids[1, 2] = 99
    coef = rng.random((M, A)).astype(np.float32)
    partial = rng.standard_normal((M * A, N)).astype(np.float32)
    y, _ = orc.combine(partial, ids, coef, E, N)
    yf = orc.bf16_to_f32(y)
    for m in (0, 2):
        v = np.zeros(N, np.float32)
        for a in range(A):  # fmaf == one rounding of the exact product-sum; float64 product then f32 round
            v = (coef[m, a].astype(np.float64) * partial[m * A + a] + v).astype(np.float32)
        assert np.array_equal(y[m], orc.f32_to_bf16(v))
    assert np.all(np.isnan(yf[1]))


def test_swiglu_bf16_form(orc):
    rng = np.random.default_rng(6)
    gu = orc.f32_to_bf16(rng.standard_normal((4, 32)).astype(np.float32) * 3)
    h = orc.swiglu_bf16(gu, 16)
    g, u = orc.bf16_to_f32(gu[:, :16]), orc.bf16_to_f32(gu[:, 16:])
    s = orc.bf16_to_f32(orc.f32_to_bf16((g / (1 + np.exp(-g))).astype(np.float32)))
    ref = orc.f32_to_bf16((s * u).astype(np.float32))
    assert np.max(np.abs(h.astype(np.int32) - ref.astype(np.int32))) <= 1  # expf ulps


# ---- the reference's F16 matrix-unit math (Q4 experts) -----------------------------------------------------------
def test_bf16_to_f16_rtz_known_answers(orc):
    b = np.array([0x3F80, 0x3EAB, 0x4789, 0xC789, 0x3580, 0x33C0, 0x33E0, 0x7F80, 0x3300, 0x0000], np.uint16)
    h = orc.bf16_to_f16_rtz(b).astype(np.float64)
    ulp = 2.0 ** -24  # F16's smallest subnormal
    want = [1.0, 0.333984375, 65504.0, -65504.0, 2.0 ** -20, ulp, ulp, np.inf, 0.0, 0.0]
    # 70144 -> 65504 (toward zero, not inf); 1.5 and 1.75 units of 2^-24 -> 1 unit (nearest-even would give 2);
    # 2^-25 -> 0
    assert list(h) == want
    assert np.isnan(orc.bf16_to_f16_rtz(np.array([0x7FC0], np.uint16))[0])
    # every BF16 in F16's normal range converts exactly
    v = orc.bf16_to_f32(np.arange(0x3880, 0x4780, dtype=np.uint16))
    assert np.array_equal(orc.bf16_to_f16_rtz(np.arange(0x3880, 0x4780, dtype=np.uint16)).astype(np.float32), v)


def test_q4_weights_f16_one_rounding(orc):
    N, K, G = 64, 256, 128
    q, s, m = orc.gen_q(4, 91, 92, N, K, G)
    w16 = orc.q4_weights_f16(q, s, m, N, K, G).astype(np.float64)
    exact = orc.dequantize(4, q, s, m, N, K, G).astype(np.float64)  # the C oracle's code * s + m (nibble order)
    # the generated scales and mins are exact in F16, so the F16 weight is the exact one rounded once to nearest
    assert np.array_equal(orc.bf16_to_f32(s).astype(np.float16).astype(np.float32), orc.bf16_to_f32(s))
    half_ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64) / 2
    assert np.all(np.abs(w16 - exact) <= half_ulp)
    assert np.array_equal(w16, exact.astype(np.float16).astype(np.float64))


def test_experts_f16math_against_exact_weights(orc):
    """The F16-math gate_up / down against the exact-weight C oracle: equal to F16 rounding (2^-9 relative on these
    sizes), and a wrong expert, slot row or operand order would be off by O(1)."""
    w, x = _tiny_layer(orc, M=6, shared=False)
    E, I = w["E"], w["I"]
    H = x.shape[1]
    ids = np.array([[0, 3], [2, 2], [1, 0], [3, 1], [0, 2], [1, 1]], np.int32)
    bits, q, s, m, G = w["gu"]
    h16 = orc.experts_gate_up_swiglu_f16math(x, bits, q, s, m, E * 2 * I, H, G, E, ids)
    h = orc.experts_gate_up_swiglu(x, orc.qview(bits, q, s, m, E * 2 * I, H, G), E, ids)
    hf, h16f = orc.bf16_to_f32(h), orc.bf16_to_f32(h16)
    assert np.abs(h16f - hf).max() <= np.abs(hf).max() * 2 ** -9
    bits, q, s, m, G = w["dn"]
    p16 = orc.experts_down_f16math(h, bits, q, s, m, E * H, I, G, E, ids)
    p = orc.experts_down(h, orc.qview(bits, q, s, m, E * H, I, G), E, ids)
    assert np.abs(p16 - p).max() <= np.abs(p).max() * 2 ** -9
    # brute force for one slot: F16 products summed in float64
    sl, e = 7, ids.ravel()[7]
    xs = orc.bf16_to_f16_rtz(h[sl]).astype(np.float64)
    w16 = orc.q4_weights_f16(q, s, m, E * H, I, G)[e * H:(e + 1) * H].astype(np.float64)
    assert np.allclose(p16[sl], [sum(xs[kk] * w16[n, kk] for kk in range(I)) for n in range(H)], rtol=1e-6, atol=1e-6)


def test_experts_gather_f16math_brute_force(orc):
    """The plain gather's F16 model at G 32 (a group every 32 k): each output the float64 sum of F16 x (toward zero)
    times the F16 weight code * f16(s) + f16(m) of that k's group, built here from the nibbles by hand; a weight
    taken from a neighbouring group, the wrong x row (slot instead of slot // A) or the high/low nibble swapped fails."""
    N, K, G, E, A = 8, 64, 32, 2, 2
    q, s, m = orc.gen_q(4, 71, 72, E * N, K, G)
    x = orc.gen_bf16_normal(73, 1.0, (3, K))
    ids = np.array([[1, 0], [0, 0], [1, 1]], np.int32)
    got = orc.experts_gather_f16math(x, 4, q, s, m, E * N, K, G, E, ids)
    xf = orc.bf16_to_f16_rtz(x).astype(np.float64)
    sf = orc.bf16_to_f32(s).astype(np.float16).astype(np.float64).reshape(E * N, K // G)
    mf = orc.bf16_to_f32(m).astype(np.float16).astype(np.float64).reshape(E * N, K // G)
    qb = np.asarray(q, np.uint8).reshape(E * N, K // 2)
    for slot in range(ids.size):
        e, row = ids.ravel()[slot], slot // A
        for n in range(N):
            r = e * N + n
            acc = 0.0
            for k in range(K):
                code = (qb[r, k // 2] >> (4 * (k % 2))) & 0xF
                w = np.float64(np.float16(code * sf[r, k // G] + mf[r, k // G]))
                acc += xf[row, k] * w
            assert abs(got[slot, n] - acc) <= 1e-6 * max(1.0, abs(acc)), (slot, n)
