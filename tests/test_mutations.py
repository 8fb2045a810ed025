"""Mutation tests of the parity checks (CPU): every plausible kernel mistake, reproduced on the oracle's side by
perturbing what a buggy kernel would have read or written, must be rejected by the very checks the GPU parity tests
apply (ids / offsets / slots bit-exact, outputs within max |got - ref| / max |ref| < 1e-2). A check that passes a
mutant would pass that bug on the GPU too.

The model is strixite's own first-kernel tutorial, which breaks its kernel on purpose to show the test catches it
(tutorial/first-kernel/first_kernel.hip:141-157); here the break is one per kernel family of the MoE path: router /
top-k, packing, gate_up + SwiGLU, down, combine, shared expert."""
import numpy as np
import pytest

TOL = 1e-2  # the layer tolerance of the GPU parity tests
# The configs' shared Q8 expert (codes uniform in [-127, 127]) has weights ~16x the routed Q4 experts' (codes - 8),
# so its term in y is ~10^3x the routed sum's and a bf16 y cannot resolve the routed experts at all. The GPU layer
# tests therefore also run each layer with the shared expert's scales and mins times SHARED_BALANCE (exact in bf16),
# which brings the two terms to the same size; the mutants below are checked on that balanced layer.
SHARED_BALANCE = 2.0 ** -4


def rel_err(got, ref):
    import oracle as orc

    g = orc.bf16_to_f32(got) if got.dtype == np.uint16 else got
    r = orc.bf16_to_f32(ref) if ref.dtype == np.uint16 else ref
    return float(np.abs(g.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def _layer(orc, M=12, H=256, E=8, k=3, I=128, seed=11):
    key = lambda t: orc.tensor_key(seed, t)  # noqa: E731
    w = {"E": E, "k": k, "I": I}
    w["router"] = orc.gen_bf16_normal(key("router"), 0.02, (E + 1, H))
    w["gu"] = (4, *orc.gen_q(4, key("gu_q"), key("gu_s"), E * 2 * I, H, 128), 128)
    w["dn"] = (4, *orc.gen_q(4, key("dn_q"), key("dn_s"), E * H, I, 128), 128)
    w["sh_gu"] = (8, *orc.gen_q(8, key("sh_gu_q"), key("sh_gu_s"), 2 * I, H, 64), 64)
    w["sh_dn"] = (8, *orc.gen_q(8, key("sh_dn_q"), key("sh_dn_s"), H, I, 64), 64)
    x = orc.gen_bf16_normal(key("x"), 1.0, (M, H))
    return w, x


def _layer_passes(orc, w, x, ref, logits_in=None):
    """The GPU tests' layer check (_layer_parity): ids bit-exact and y within TOL."""
    o = orc.moe_layer(w, x, logits_in=logits_in)
    return np.array_equal(o["ids"], ref["ids"]) and rel_err(o["y"], ref["y"]) < TOL


def _with(w, name, q=None, s=None, m=None):
    bits, q0, s0, m0, G = w[name]
    w2 = dict(w)
    w2[name] = (bits, q0 if q is None else q, s0 if s is None else s, m0 if m is None else m, G)
    return w2


def balanced(orc, w):
    """The shared expert's scales and mins times SHARED_BALANCE (a power of two: exact on bf16 bits)."""
    w2 = dict(w)
    for name in ("sh_gu", "sh_dn"):
        bits, q, s, m, G = w[name]
        sc = lambda b: orc.f32_to_bf16(orc.bf16_to_f32(b) * np.float32(SHARED_BALANCE))  # noqa: E731
        w2[name] = (bits, q, sc(s), sc(m), G)
    return w2


@pytest.fixture(scope="module")
def case(orc):
    w, x = _layer(orc)
    w = balanced(orc, w)
    return w, x, orc.moe_layer(w, x)


def test_config_scale_shared_expert_hides_routed_bugs(orc):
    """Why the balanced pass exists: at the configs' scales a routed-expert bug (the min term dropped) stays inside
    the layer tolerance, while the balanced layer rejects it."""
    w, x = _layer(orc)
    ref = orc.moe_layer(w, x)
    bad = _with(w, "gu", m=np.zeros_like(w["gu"][3]))
    assert _layer_passes(orc, bad, x, ref)  # invisible at the configs' shared-expert scale
    wb = balanced(orc, w)
    assert not _layer_passes(orc, _with(wb, "gu", m=np.zeros_like(w["gu"][3])), x, orc.moe_layer(wb, x))


def test_unmutated_layer_passes(orc, case):
    w, x, ref = case
    assert _layer_passes(orc, w, x, ref)


# ---- router / top-k ----------------------------------------------------------------------------------------------
def test_router_reading_the_wrong_expert_row_is_caught(orc, case):
    """The router projection's row index off by one (expert e's logit from row e + 1)."""
    w, x, ref = case
    E = w["E"]
    r = w["router"].copy()
    r[:E] = np.roll(r[:E], -1, axis=0)
    w2 = dict(w, router=r)
    assert not _layer_passes(orc, w2, x, ref)


def test_topk_tie_to_the_higher_index_is_caught(orc):
    """Ties broken toward the higher expert index instead of the lower (strixite kernels/moe_router.hip:88)."""
    E, k = 16, 4
    lg = np.zeros((3, E), np.float32)
    lg[:, 3] = lg[:, 9] = 1.0  # a tie for the top pick
    lg[:, 5] = 0.5
    ids, _, _ = orc.topk(lg, E, k)
    wrong = ids.copy()
    wrong[:, [0, 1]] = wrong[:, [1, 0]]  # 9 before 3
    assert list(ids[0, :2]) == [3, 9]
    assert not np.array_equal(wrong, ids)


def test_topk_softmax_over_all_experts_is_caught(orc, case):
    """Softmax over all E logits instead of the k picks: the coefficients differ beyond the tests' rtol 2e-6."""
    w, x, ref = case
    E, k = w["E"], w["k"]
    lg = ref["logits"][:, :E].astype(np.float64)
    full = np.exp(lg - lg.max(1, keepdims=True))
    full /= full.sum(1, keepdims=True)
    wrong = np.take_along_axis(full, ref["ids"][:, :k].astype(np.int64), 1).astype(np.float32)
    assert not np.allclose(wrong, ref["coef"][:, :k], rtol=2e-6, atol=1e-7)


# ---- packing -----------------------------------------------------------------------------------------------------
def test_unstable_bucket_order_and_wrong_offsets_are_caught(orc, case):
    """Slots of a bucket in descending instead of ascending order; offsets shifted by one bucket."""
    w, x, ref = case
    offsets, slots, _ = orc.group_routes(ref["ids"], w["E"])
    bad = slots.copy()
    for b in range(w["E"]):
        lo, hi = offsets[b], offsets[b + 1]
        bad[lo:hi] = bad[lo:hi][::-1]
    assert np.array_equal(offsets, ref["offsets"])
    assert not np.array_equal(bad, slots)
    assert not np.array_equal(np.roll(offsets, 1), offsets)


# ---- gate_up + SwiGLU --------------------------------------------------------------------------------------------
def _gu_rows(w):
    bits, q, s, m, G = w["gu"]
    E, I = w["E"], w["I"]
    H = q.size * 2 // (E * 2 * I)
    return q.reshape(E, 2, I, H // 2), s.reshape(E, 2, I, H // G), m.reshape(E, 2, I, H // G)


def test_gate_and_up_swapped_is_caught(orc, case):
    """The gate and up halves exchanged (silu applied to u): a transposed operand role."""
    w, x, ref = case
    q, s, m = _gu_rows(w)
    w2 = _with(w, "gu", q=np.ascontiguousarray(q[:, ::-1]).ravel(), s=np.ascontiguousarray(s[:, ::-1]).ravel(),
               m=np.ascontiguousarray(m[:, ::-1]).ravel())
    assert not _layer_passes(orc, w2, x, ref)


def test_tile_offset_by_16_rows_is_caught(orc, case):
    """A 16-row weight tile read 16 rows late (a wrong tile offset inside an expert)."""
    w, x, ref = case
    q, s, m = _gu_rows(w)
    w2 = _with(w, "gu", q=np.roll(q, -16, axis=2).ravel(), s=np.roll(s, -16, axis=2).ravel(),
               m=np.roll(m, -16, axis=2).ravel())
    assert not _layer_passes(orc, w2, x, ref)


def test_expert_stride_off_by_one_expert_is_caught(orc, case):
    """Expert e's weights read from expert e + 1's rows (a wrong expert base)."""
    w, x, ref = case
    q, s, m = _gu_rows(w)
    w2 = _with(w, "gu", q=np.roll(q, -1, axis=0).ravel(), s=np.roll(s, -1, axis=0).ravel(),
               m=np.roll(m, -1, axis=0).ravel())
    assert not _layer_passes(orc, w2, x, ref)


def test_nibble_order_swapped_is_caught(orc, case):
    """Q4 codes decoded high nibble first (code 2j from the high nibble)."""
    w, x, ref = case
    q = w["gu"][1]
    w2 = _with(w, "gu", q=((q >> 4) | (q << 4)).astype(np.uint8))
    assert not _layer_passes(orc, w2, x, ref)


def test_dropped_min_term_is_caught(orc, case):
    """The min term (m * sum x over the group) left out of the accumulator."""
    w, x, ref = case
    m = w["gu"][3]
    w2 = _with(w, "gu", m=np.zeros_like(m))
    assert not _layer_passes(orc, w2, x, ref)


def test_last_quantization_group_dropped_is_caught(orc, case):
    """A K loop one group short (the last quantization group of every row missing)."""
    w, x, ref = case
    _, _, s, m, G = w["gu"]
    ng = x.shape[1] // G
    s2, m2 = s.reshape(-1, ng).copy(), m.reshape(-1, ng).copy()
    s2[:, -1] = 0
    m2[:, -1] = 0
    w2 = _with(w, "gu", s=s2.ravel(), m=m2.ravel())
    assert not _layer_passes(orc, w2, x, ref)


# ---- down --------------------------------------------------------------------------------------------------------
def test_down_reading_the_neighbour_slot_is_caught(orc, case):
    """The down projection fed slot s + 1's h row."""
    w, x, ref = case
    E, I = w["E"], w["I"]
    H = x.shape[1]
    bits, q, s, m, G = w["dn"]
    view = orc.qview(bits, q, s, m, (E + 0) * H, I, G)
    ids = ref["ids"]
    good = orc.experts_down(ref["h"], view, E, ids)
    bad = orc.experts_down(np.ascontiguousarray(np.roll(ref["h"], 1, axis=0)), view, E, ids)
    assert rel_err(good, ref["partial"]) < TOL
    assert rel_err(bad, ref["partial"]) >= TOL


# ---- combine -----------------------------------------------------------------------------------------------------
def test_combine_coefficients_of_the_wrong_slot_are_caught(orc, case):
    """The ordered sum weighting slot a's partial with slot a + 1's coefficient."""
    w, x, ref = case
    E, H = w["E"], x.shape[1]
    y, _ = orc.combine(ref["partial"], ref["ids"], np.ascontiguousarray(np.roll(ref["coef"], 1, axis=1)), E, H)
    y0, _ = orc.combine(ref["partial"], ref["ids"], ref["coef"], E, H)
    assert rel_err(y, y0) >= TOL


def test_shared_gate_without_sigmoid_is_caught(orc, case):
    """The shared expert added with weight 1 instead of sigmoid(its gate logit)."""
    w, x, ref = case
    E, H = w["E"], x.shape[1]
    gl = np.ascontiguousarray(ref["logits"][:, E:E + 1])  # the shared gate logit, column E
    big = np.full_like(gl, 50.0)  # sigmoid -> 1
    y, _ = orc.combine(ref["partial"], ref["ids"], ref["coef"], E, H, s=ref["sh_s"], gate_logit=big, gate_ld=1)
    y0, _ = orc.combine(ref["partial"], ref["ids"], ref["coef"], E, H, s=ref["sh_s"], gate_logit=gl, gate_ld=1)
    assert rel_err(y0, ref["y"]) < TOL
    assert rel_err(y, y0) >= TOL


def test_shared_down_rows_reversed_is_caught(orc, case):
    """The shared expert's down rows indexed from the wrong end (output n from weight row H - 1 - n)."""
    w, x, ref = case
    bits, q, s, m, G = w["sh_dn"]
    H, I = x.shape[1], w["I"]
    w2 = _with(w, "sh_dn", q=np.ascontiguousarray(q.reshape(H, I)[::-1]).ravel(),
               s=np.ascontiguousarray(s.reshape(H, I // G)[::-1]).ravel(),
               m=np.ascontiguousarray(m.reshape(H, I // G)[::-1]).ravel())
    assert not _layer_passes(orc, w2, x, ref)
