"""Host-side mirror of strixite's MoE launch interface over the gfx950 library, on torch device tensors.

The names, argument meanings and error behaviour follow the reference's launchers (strixite
``kernels/moe_router.hpp``, ``kernels/moe_grouped.hpp``, ``kernels/linear_q4.hpp``, ``kernels/swiglu.hpp``,
``kernels/linear_q8.hpp``, ``kernels/linear.hpp``); each function forwards to the C-ABI entry point of the same name
(include/strixite_moe.h). torch supplies device memory and the current stream only; all arithmetic runs in the HIP
kernels. A failed precondition raises StrixError, a HIP failure GpuError; device-detected data errors set the err
words (3 x uint32, first flag wins) and NaN the affected rows, as in the reference.
"""
from __future__ import annotations

from dataclasses import dataclass

import ctypes as C
import torch

from . import _lib as L
from ._lib import GpuError, StrixError  # noqa: F401  (re-exported)

F32, BF16 = 0, 1
# strixite MoeMath (kernels/moe_grouped.hpp:39): the F16 kinds (2..5) run Q4 experts' grouped projections in the
# reference's F16 math (x and the dequantized weights in F16) at every batch size; F32 and WmmaBf16 keep the weights
# exact (and take the decode-size stream kernels)
MOE_MATH_F32, MOE_MATH_WMMA_BF16, MOE_MATH_WMMA_F16 = 0, 1, 2

TENSOR = {  # tensor ids of the seeded generator (oracle/moe_oracle.c uses the same ids)
    "x": 1, "router": 2, "gu_q": 3, "gu_s": 4, "dn_q": 5, "dn_s": 6,
    "sh_gu_q": 7, "sh_gu_s": 8, "sh_dn_q": 9, "sh_dn_s": 10, "logits": 11, "zipf": 12,
}


def _p(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _act_dtype(t: torch.Tensor) -> torch.dtype:
    """The activation dtype of the outputs that follow input t: FP32 for an FP32 input, BF16 otherwise."""
    return torch.float32 if t.dtype == torch.float32 else torch.bfloat16


def _act(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise StrixError(f"activation dtype {t.dtype} unsupported (float32 or bfloat16)")


def zero_err(device="cuda") -> torch.Tensor:
    return torch.zeros(3, dtype=torch.int32, device=device)


# ---- weights ---------------------------------------------------------------------------------------------------
@dataclass
class QWeight:
    """A Q4 / Q8 weight on the device (strixite formats/q4.hpp, formats/q8.hpp layouts): q [N, K/2] or [N, K] bytes,
    scale / minv [N, K/G] bf16 bits (int16 storage), w = q * scale + minv."""
    bits: int
    q: torch.Tensor
    scale: torch.Tensor
    minv: torch.Tensor
    N: int
    K: int
    G: int

    def view(self) -> L.QView:
        return L.QView(_p(self.q), _p(self.scale), _p(self.minv), self.N, self.K, self.G)

    @property
    def nbytes(self) -> int:
        return self.q.numel() + 2 * self.scale.numel() + 2 * self.minv.numel()

    @staticmethod
    def empty(bits: int, N: int, K: int, G: int, device="cuda") -> "QWeight":
        q = torch.empty(N * K // (2 if bits == 4 else 1), dtype=torch.uint8, device=device)
        s = torch.empty(N * (K // G), dtype=torch.int16, device=device)
        m = torch.empty_like(s)
        return QWeight(bits, q, s, m, N, K, G)

    @staticmethod
    def from_host(bits, q, s, m, N, K, G, device="cuda") -> "QWeight":
        """From numpy arrays (uint8 codes, uint16 bf16 bits)."""
        import numpy as np

        return QWeight(bits, torch.from_numpy(np.ascontiguousarray(q)).to(device),
                       torch.from_numpy(np.ascontiguousarray(s).view(np.int16)).to(device),
                       torch.from_numpy(np.ascontiguousarray(m).view(np.int16)).to(device), N, K, G)

    @staticmethod
    def synth(bits: int, seed: int, codes: str, scales: str, layer: int, N: int, K: int, G: int,
              device="cuda") -> "QWeight":
        """Seeded synthetic weight generated on the device (codes uniform, scale bf16(|N(0,0.02)|), min -8s or
        -128s)."""
        w = QWeight.empty(bits, N, K, G, device)
        kc, ks = synth_key(seed, codes, layer), synth_key(seed, scales, layer)
        L.check(L.lib().strix_synth_q_weight(bits, kc, ks, N, K, G, _p(w.q), _p(w.scale), _p(w.minv), _stream()))
        return w


def synth_key(seed: int, tensor: str | int, layer: int = 0) -> int:
    t = TENSOR[tensor] if isinstance(tensor, str) else tensor
    return int(L.lib().strix_synth_tensor_key(seed, t, layer))


def synth_bf16_normal(seed: int, tensor: str, layer: int, shape, sigma: float, device="cuda") -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    L.check(L.lib().strix_synth_bf16_normal(synth_key(seed, tensor, layer), sigma, _p(out), out.numel(), _stream()))
    return out


def synth_uniform_pm1(seed: int, tensor: str, layer: int, shape, device="cuda") -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float32, device=device)
    L.check(L.lib().strix_synth_uniform_pm1(synth_key(seed, tensor, layer), _p(out), out.numel(), _stream()))
    return out


# ---- router ----------------------------------------------------------------------------------------------------
def linear_bf16w(x: torch.Tensor, w: torch.Tensor, out_dtype=torch.float32, y: torch.Tensor | None = None):
    """strixite kernels/linear.hpp:23-26: y = x W^T, FP32 accumulation in one fixed order."""
    M, K = x.shape
    N = w.shape[0]
    if y is None:
        y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    L.check(L.lib().strix_linear_bf16w(_p(x), _p(w), _p(y), M, N, K, _act(x), _act(y), _stream()))
    return y


def moe_router(logits: torch.Tensor, E: int, k: int, shared_logit: torch.Tensor | None = None, shared_ld: int = 1,
               shared_id: int = 0, err: torch.Tensor | None = None, ld: int | None = None, M: int | None = None):
    """strixite kernels/moe_router.hpp:38-40. Returns (ids [M, A] int32, coef [M, A] f32, err)."""
    M = M if M is not None else logits.shape[0]
    ld = ld if ld is not None else logits.shape[-1]
    A = k + (1 if shared_logit is not None else 0)
    ids = torch.empty((M, A), dtype=torch.int32, device=logits.device)
    coef = torch.empty((M, A), dtype=torch.float32, device=logits.device)
    err = zero_err(logits.device) if err is None else err
    L.check(L.lib().strix_moe_router(_p(logits), ld, M, E, k, _p(shared_logit), shared_ld, shared_id, _p(ids),
                                     _p(coef), _act(logits), _p(err), _stream()))
    return ids, coef, err


def check_router_error(err: torch.Tensor, what: str = "moe_router") -> None:
    L.check(L.lib().strix_check_router_error(_p(err), what.encode()))


def check_expert_error(err: torch.Tensor, what: str = "experts") -> None:
    L.check(L.lib().strix_check_expert_error(_p(err), what.encode()))


def moe_shared_add(y, s, gate_logit, gate_ld, gate_index, err):
    M, N = y.shape
    L.check(L.lib().strix_moe_shared_add(_p(y), _p(s), _p(gate_logit), gate_ld, M, N, gate_index, _act(y), _p(err),
                                         _stream()))


def moe_shared_add_inject(y, s, gate_logit, gate_ld, gate_index, x, w_in, H, err):
    M, N = y.shape
    L.check(L.lib().strix_moe_shared_add_inject(_p(y), _p(s), _p(gate_logit), gate_ld, M, N, gate_index, _p(x),
                                                _p(w_in), H, _act(y), _p(err), _stream()))


# ---- grouping --------------------------------------------------------------------------------------------------
def moe_route_workspace_bytes(M: int, A: int, E: int) -> int:
    n = L.lib().strix_moe_route_workspace_bytes(M, A, E)
    if n < 0:
        L.check(1)
    return n


def moe_group_routes(ids: torch.Tensor, E: int, ws: torch.Tensor | None = None, err: torch.Tensor | None = None):
    """strixite kernels/moe_grouped.hpp:52-53. Returns (ws int32, err)."""
    if ids.dtype != torch.int32 or ids.dim() != 2 or not ids.is_contiguous():
        raise TypeError(f"moe_group_routes: ids must be a contiguous [M, A] int32 tensor, got {ids.dtype} "
                        f"{tuple(ids.shape)}")
    M, A = ids.shape
    nbytes = moe_route_workspace_bytes(M, A, E)
    if ws is None:
        ws = torch.empty(nbytes // 4, dtype=torch.int32, device=ids.device)
    err = zero_err(ids.device) if err is None else err
    L.check(L.lib().strix_moe_group_routes(_p(ids), M, A, E, _p(ws), ws.numel() * 4, _p(err), _stream()))
    return ws, err


def route_tables(ws: torch.Tensor, M: int, A: int, E: int) -> dict:
    """The reference's prefix of the grouping workspace: header, offsets [E + 2], slots [S]."""
    S = M * A
    return {"n_tiles": ws[0], "S": ws[1], "E": ws[2], "offsets": ws[4:4 + E + 2], "slots": ws[4 + E + 2:4 + E + 2 + S]}


# ---- experts ---------------------------------------------------------------------------------------------------
def _fam(bits):
    """The C-ABI family of a weight format: q4, q5 (formats/q5.hpp) or q8."""
    return {4: "q4", 5: "q5", 8: "q8"}[bits]


def _swiglu_fn(bits):
    return getattr(L.lib(), f"strix_linear_{_fam(bits)}_experts_gather_grouped_swiglu")


def _combine_fn(bits):
    return getattr(L.lib(), f"strix_linear_{_fam(bits)}_experts_combine_grouped")


def experts_gather_grouped_swiglu(x, w: QWeight, E, ws, M, A, h_f16=False, h=None, math=MOE_MATH_WMMA_F16):
    """strixite kernels/moe_grouped.hpp:66-69 (Q4; Q8 through the same signature family)."""
    I = w.N // E // 2
    if h is None:
        h = torch.empty((M * A, I), dtype=torch.float16 if h_f16 else _act_dtype(x), device=x.device)
    v = w.view()
    L.check(_swiglu_fn(w.bits)(_p(x), C.byref(v), E, _p(ws), ws.numel() * 4, M, A, _p(h), _act(x), math, _stream(),
                               1 if h_f16 else 0))
    return h


def experts_gather_grouped(x, w: QWeight, E, ws, M, A, y=None, math=MOE_MATH_WMMA_F16):
    """strixite kernels/moe_grouped.hpp:56-58: y [M * A, N] = x[slot / A] W[id]^T (Q4)."""
    N = w.N // E
    if y is None:
        y = torch.empty((M * A, N), dtype=_act_dtype(x), device=x.device)
    v = w.view()
    L.check(getattr(L.lib(), f"strix_linear_{_fam(w.bits)}_experts_gather_grouped")(
        _p(x), C.byref(v), E, _p(ws), ws.numel() * 4, M, A, _p(y),
                                                           _act(x), math, _stream()))
    return y


def experts_combine_grouped(h, w: QWeight, E, ids, coef, ws, M, A, partial=None, y=None, shared: dict | None = None,
                            h_f16=False, math=MOE_MATH_WMMA_F16):
    """strixite kernels/moe_grouped.hpp:88-91 (+ MoeSharedAdd). Returns y [M, N]."""
    N = w.N // E
    if partial is None:
        partial = torch.empty((M * A, N), dtype=torch.float32, device=h.device)
    if y is None:
        y = torch.empty((M, N), dtype=_act_dtype(h), device=h.device)
    sh = None
    if shared is not None:
        sh = L.SharedAdd(_p(shared["s"]), _p(shared["gate_logit"]), shared["gate_ld"], shared["gate_index"],
                         _p(shared["err"]))
    v = w.view()
    L.check(_combine_fn(w.bits)(_p(h), C.byref(v), E, _p(ids), _p(coef), _p(ws), ws.numel() * 4, _p(partial), M, A,
                                _p(y), _act(h) if not h_f16 else BF16, math, _stream(), C.byref(sh) if sh is not None else None,
                                1 if h_f16 else 0))
    return y


def experts_gather(x, w: QWeight, E, ids, err, swiglu=False):
    """strixite kernels/linear_q4.hpp:42-43 / 55-56 (per-slot)."""
    M, A = ids.shape
    N = w.N // E
    y = torch.empty((M * A, N // 2 if swiglu else N), dtype=_act_dtype(x), device=x.device)
    fam = _fam(w.bits)
    fn = getattr(L.lib(), f"strix_linear_{fam}_experts_gather_swiglu" if swiglu else f"strix_linear_{fam}_experts_gather")
    v = w.view()
    L.check(fn(_p(x), C.byref(v), E, _p(ids), M, A, _p(y), _act(x), _p(err), _stream()))
    return y


def experts_combine(h, w: QWeight, E, ids, coef, err):
    """strixite kernels/linear_q4.hpp:44-46 (per-slot)."""
    M, A = ids.shape
    N = w.N // E
    y = torch.empty((M, N), dtype=_act_dtype(h), device=h.device)
    v = w.view()
    L.check(getattr(L.lib(), f"strix_linear_{_fam(w.bits)}_experts_combine")(_p(h), C.byref(v), E, _p(ids), _p(coef), M, A, _p(y), _act(h),
                                                    _p(err), _stream()))
    return y


def swiglu(gu: torch.Tensor, I: int) -> torch.Tensor:
    """strixite kernels/swiglu.hpp:21."""
    rows = gu.numel() // (2 * I)
    h = torch.empty((rows, I), dtype=gu.dtype, device=gu.device)
    L.check(L.lib().strix_swiglu(_p(gu), _p(h), rows, I, _act(gu), _stream()))
    return h


def linear_q8(x: torch.Tensor, w: QWeight, out_dtype=torch.bfloat16) -> torch.Tensor:
    """strixite kernels/linear_q8.hpp:13-14."""
    M = x.shape[0]
    y = torch.empty((M, w.N), dtype=out_dtype, device=x.device)
    v = w.view()
    L.check(L.lib().strix_linear_q8(_p(x), C.byref(v), _p(y), M, _act(x), _act(y), _stream()))
    return y


def linear_q4(x: torch.Tensor, w: QWeight, out_dtype=torch.bfloat16) -> torch.Tensor:
    """strixite kernels/linear_q4.hpp:23-31."""
    M = x.shape[0]
    y = torch.empty((M, w.N), dtype=out_dtype, device=x.device)
    v = w.view()
    L.check(L.lib().strix_linear_q4(_p(x), C.byref(v), _p(y), M, _act(x), _act(y), _stream()))
    return y


def hc_inject(x: torch.Tensor, w_in: torch.Tensor, y: torch.Tensor) -> None:
    """strixite kernels/hc.hpp:51-55, in place: x [T, H d] += w_in [T, H] * y [T, d] per stream, one rounding."""
    T, Hd = x.shape
    H = w_in.shape[1]
    L.check(L.lib().strix_hc_inject(_p(x), _p(w_in), _p(y), T, H, Hd // H, _act(x), _stream()))


# ---- the sublayer ----------------------------------------------------------------------------------------------
class LayerContext:
    """The helper stream (and its fork / join events) on which the sublayer runs the shared expert beside the routing
    kernels at prefill sizes (strix_moe_layer_context_create). Create it before any graph capture, on the device it
    serves; use it from one thread at a time."""

    def __init__(self):
        h = C.c_void_p()
        L.check(L.lib().strix_moe_layer_context_create(C.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            L.lib().strix_moe_layer_context_destroy(self._h)
            self._h = None


class MoeLayer:
    """One MoE FFN sublayer's weights on the device and its forward (strixite runtime/qwen4exp.cpp:3143-3217)."""

    def __init__(self, H, E, k, I, router, gate_up: QWeight, down: QWeight, router_bias=None,
                 shared_gate_up: QWeight | None = None, shared_down: QWeight | None = None,
                 shared_stacked: bool = False):
        """shared_stacked: the shared expert is expert E of gate_up / down (E + 1 experts there, router row E its
        gate), routed as slot k of every token; ids / coef are then [M, k + 1]."""
        self.H, self.E, self.k, self.I = H, E, k, I
        self.shared_stacked = shared_stacked
        self.A = k + (1 if shared_stacked else 0)
        self.router, self.router_bias = router, router_bias
        self.gate_up, self.down = gate_up, down
        self.shared_gate_up, self.shared_down = shared_gate_up, shared_down
        self._w = L.LayerWeights()
        w = self._w
        w.H, w.E, w.k, w.I = H, E, k, I
        w.router = _p(router)
        w.router_bias = _p(router_bias)
        w.routed_bits = gate_up.bits
        w.gate_up, w.down = gate_up.view(), down.view()
        w.has_shared = 1 if shared_gate_up is not None else 0
        if shared_gate_up is not None:
            w.sh_gate_up, w.sh_down = shared_gate_up.view(), shared_down.view()
        w.shared_stacked = 1 if shared_stacked else 0

    @staticmethod
    def from_view(w: "L.LayerWeights", owner=None) -> "MoeLayer":
        """A layer over weights that live elsewhere in device memory (e.g. a strixw file loaded into HBM); owner is
        kept alive with the layer."""
        m = MoeLayer.__new__(MoeLayer)
        m.H, m.E, m.k, m.I = w.H, w.E, w.k, w.I
        m.shared_stacked = bool(w.shared_stacked)
        m.A = m.k + (1 if m.shared_stacked else 0)
        m.router = m.router_bias = m.gate_up = m.down = m.shared_gate_up = m.shared_down = None
        m._has_shared_view = bool(w.has_shared)
        m._owner = owner
        m._w = w
        return m

    @property
    def has_shared(self) -> bool:
        return getattr(self, "_has_shared_view", False) or self.shared_gate_up is not None

    @property
    def weight_bytes(self) -> int:
        n = self.gate_up.nbytes + self.down.nbytes + (self.router.numel() * 2 if self.router is not None else 0)
        if self.has_shared:
            n += self.shared_gate_up.nbytes + self.shared_down.nbytes
        return n

    @staticmethod
    def synth(H, E, k, I, seed=0, layer=0, routed_bits=4, routed_G=None, shared=True, shared_G=64,
              router_bias=None, device="cuda") -> "MoeLayer":
        """Seeded synthetic layer (router N(0, 0.02), Q4 / Q8 experts as the bench configs describe). shared: True (a
        separate Q8 shared expert), False, or "stacked" (the shared expert as expert E of the routed stacks)."""
        G = routed_G or (128 if routed_bits == 4 else 64)
        stacked = shared == "stacked"
        Es = E + (1 if stacked else 0)
        router = synth_bf16_normal(seed, "router", layer, (E + (1 if shared else 0), H), 0.02, device)
        gu = QWeight.synth(routed_bits, seed, "gu_q", "gu_s", layer, Es * 2 * I, H, G, device)
        dn = QWeight.synth(routed_bits, seed, "dn_q", "dn_s", layer, Es * H, I, G, device)
        if stacked:
            return MoeLayer(H, E, k, I, router, gu, dn, router_bias, shared_stacked=True)
        sgu = sdn = None
        if shared:
            sgu = QWeight.synth(8, seed, "sh_gu_q", "sh_gu_s", layer, 2 * I, H, shared_G, device)
            sdn = QWeight.synth(8, seed, "sh_dn_q", "sh_dn_s", layer, H, I, shared_G, device)
        return MoeLayer(H, E, k, I, router, gu, dn, router_bias, sgu, sdn)

    def workspace_bytes(self, M: int) -> int:
        n = L.lib().strix_moe_layer_workspace_bytes(C.byref(self._w), M)
        if n < 0:
            L.check(1)
        return n

    def workspace(self, M: int, device="cuda") -> torch.Tensor:
        return torch.empty(self.workspace_bytes(M), dtype=torch.uint8, device=device)

    def forward(self, x: torch.Tensor, logits_in: torch.Tensor | None = None, ws: torch.Tensor | None = None,
                out: dict | None = None, ctx: LayerContext | None = None, inject: tuple | None = None) -> dict:
        """Returns {y, x_out, ids, coef, err[6]} (asynchronous; the tensors are filled on the current stream). ctx: a
        LayerContext for the shared expert's helper stream at prefill sizes (None: it runs on the current stream).
        inject: (xs [M, streams * H] bf16, w_in [M, streams] f32): the hyper-connection injection into xs in place,
        instead of the x_out residual write."""
        M = x.shape[0]
        if ws is None:
            ws = self.workspace(M, x.device)
        inj = None
        if inject is not None:
            xs, w_in = inject
            inj = L.InjectArgs(_p(xs), _p(w_in), w_in.shape[1])
        if out is None:
            out = {
                "y": torch.empty((M, self.H), dtype=torch.bfloat16, device=x.device),
                "x_out": torch.empty((M, self.H), dtype=torch.bfloat16, device=x.device),
                "ids": torch.empty((M, self.A), dtype=torch.int32, device=x.device),
                "coef": torch.empty((M, self.A), dtype=torch.float32, device=x.device),
                "err": torch.zeros(6, dtype=torch.int32, device=x.device),
            }
        L.check(L.lib().strix_moe_layer_forward(C.byref(self._w), _p(x), M, _p(logits_in), _p(out["y"]),
                                                _p(out["x_out"]) if inj is None else None, _p(out["ids"]),
                                                _p(out["coef"]), _p(ws), ws.numel(),
                                                _p(out["err"]), _stream(), ctx.handle if ctx is not None else None,
                                                C.byref(inj) if inj is not None else None))
        return out


# ---- hyper-connection mix: strixite kernels/hc.hpp:31-50 ----------------------------------------------------------
def hc_mix_down(x: torch.Tensor, w: QWeight, r: int, inject: bool, eps: float):
    """strixite kernels/hc.hpp:31-36: x [T, 4 d] (F32 or BF16) with the folded w [r (+ 4), 4 d] (row-major Q4 / Q8)
    -> (h [T, r], w_in [T, 4] or None, inv [T, 4]), FP32."""
    T, Hd = x.shape
    H = 4
    h = torch.empty((T, r), dtype=torch.float32, device=x.device)
    w_in = torch.empty((T, H), dtype=torch.float32, device=x.device) if inject else None
    inv = torch.empty((T, H), dtype=torch.float32, device=x.device)
    v = w.view()
    L.check(L.lib().strix_hc_mix_down(_p(x), C.byref(v), w.bits, T, H, Hd // H, r, int(inject), eps, _p(h), _p(w_in),
                                      _p(inv), _act(x), _stream()))
    return h, w_in, inv


def hc_mix_up(h: torch.Tensor, w_up: QWeight, x: torch.Tensor, norm_w: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """strixite kernels/hc.hpp:38-50: w_up [4 d, r] in the chunk-major layout (the QWeight's arrays hold it) -> u
    [T, d] in x's dtype."""
    T, Hd = x.shape
    H = 4
    u = torch.empty((T, Hd // H), dtype=x.dtype, device=x.device)
    v = w_up.view()
    L.check(L.lib().strix_hc_mix_up(_p(h), C.byref(v), w_up.bits, _p(x), _p(norm_w), _p(inv), T, H, Hd // H, _p(u),
                                    _act(x), _stream()))
    return u
