"""Shared helpers of the GPU parity tests: seeded layers built on the device through the product's generator,
their weights copied to the host for the CPU oracle, and the comparison metrics."""
import numpy as np
import torch

import oracle as orc
from strixite_amd import moe


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int16:
        return t.numpy().view(np.uint16)
    return t.numpy()


def qspec(w: moe.QWeight):
    return (w.bits, to_np(w.q), to_np(w.scale), to_np(w.minv), w.G)


def oracle_weights(layer: moe.MoeLayer) -> dict:
    w = {"E": layer.E, "k": layer.k, "I": layer.I, "router": to_np(layer.router), "gu": qspec(layer.gate_up),
         "dn": qspec(layer.down)}
    if layer.router_bias is not None:
        w["router_bias"] = to_np(layer.router_bias)
    if layer.has_shared:
        w["sh_gu"], w["sh_dn"] = qspec(layer.shared_gate_up), qspec(layer.shared_down)
    if layer.shared_stacked:
        w["shared_stacked"] = True
    return w


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (normwise; the layer tolerance is 1e-2 in bf16)."""
    g = orc.bf16_to_f32(got) if got.dtype == np.uint16 else got
    r = orc.bf16_to_f32(ref) if ref.dtype == np.uint16 else ref
    return float(np.abs(g.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def zipf_bias(seed: int, E: int, beta: float, s: float = 1.1) -> np.ndarray:
    """b_e = -beta * s * ln(rank_e) over a seeded permutation of the experts (host-side, float64 then float32)."""
    rng = np.random.default_rng(orc.tensor_key(seed, "zipf") & 0xFFFFFFFF)
    rank = rng.permutation(E) + 1
    return (-beta * s * np.log(rank.astype(np.float64))).astype(np.float32)


# The configs' shared Q8 expert (codes uniform in [-127, 127]) outweighs the routed Q4 experts ~16x per projection,
# so its term in y is ~10^3x the routed sum's and a bf16 y cannot resolve the routed experts. Layer tests therefore
# also run each layer with the shared expert's scales and mins times SHARED_BALANCE (exact on bf16 bits), which
# brings the two terms to the same size (tests/test_mutations.py shows a routed bug that only this pass catches).
SHARED_BALANCE = 2.0 ** -4


def balanced(layer: moe.MoeLayer) -> moe.MoeLayer:
    """The same layer (same routed weights, router and bias tensors) with the separate shared expert's scales and
    mins scaled by SHARED_BALANCE."""
    assert layer.shared_gate_up is not None, "balanced(): a layer with a separate shared expert"

    def sc(w: moe.QWeight) -> moe.QWeight:
        f = lambda t: (t.view(torch.bfloat16) * SHARED_BALANCE).view(torch.int16)  # noqa: E731
        return moe.QWeight(w.bits, w.q, f(w.scale), f(w.minv), w.N, w.K, w.G)

    return moe.MoeLayer(layer.H, layer.E, layer.k, layer.I, layer.router, layer.gate_up, layer.down,
                        layer.router_bias, sc(layer.shared_gate_up), sc(layer.shared_down))
