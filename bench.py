"""Benchmark of the MoE FFN sublayer on one MI355X. Prints ONE JSON line.

`value` is BASELINE config 2: a 16-token decode step (2 slots x (1 + 7 MTP drafts)) through one MoE sublayer, H 3072,
512 experts, top-10 + one shared Q8 expert, I 512, Q4 g128 routed experts. The other configs ride along in the same
line: config 4 (4096-token Zipf prefill), config 1 (1-token Q8 decode), config 3 (512-token prefill with uniform
router logits), config 5 (an 8-layer stack run as a 16-token decode step and a 4096-token prefill step back to back).

A step is one sublayer forward (router projection -> top-k -> packing -> gate_up + SwiGLU -> down -> ordered combine +
shared expert -> residual) over one batch. Every config rotates over a stack of layers with independent weights (the
bytes a rotation touches exceed the 256 MB MALL several times over); the first n layers of a rotation are captured as
one HIP graph for each n, and K steps replay the whole rotation K // L times, then the first K % L layers. Timing: `--samples` samples of exactly `--steps` steps each, bracketed by device
synchronization, HIP events on the launch stream; the median sample is reported. Inputs and weights are resident in
HBM before the timed region.

The dominant kernel of a config (decode: the grouped gate_up + SwiGLU; prefill: the F16-math grouped gate_up) is
timed alone with HIP events over its own launches and converted to a roofline fraction. The CPU oracle
(multithreaded C, oracle/) is timed on the host cores beside it, on the full config-2 layer and on a token sample of
config 4.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/s; achieved HBM GB/s (decode) and MFMA % of peak (prefill)"
PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # dense fp16 / bf16 MFMA

H, E, K_TOP, I = 3072, 512, 10, 512
GU_BYTES_PER_EXPERT = 2 * I * H // 2 + 2 * I * (H // 128) * 4    # Q4 g128 gate_up: 1,671,168 B
DN_BYTES_PER_EXPERT = H * I // 2 + H * (I // 128) * 4            # Q4 g128 down: 835,584 B
SH_BYTES = 2 * I * H + 2 * I * (H // 64) * 4 + H * I + H * (I // 64) * 4  # Q8 g64 shared: 5,013,504 B
ROUTER_BYTES = (E + 1) * H * 2
ZIPF_BETA = 1.0
# config 1: H 2048, 64 experts, top-8, I 512, Q8 g64 routed, no shared expert
C1_H, C1_E, C1_K = 2048, 64, 8
C1_BYTES_PER_EXPERT = (2 * I * C1_H + 2 * I * (C1_H // 64) * 4) + (C1_H * I + C1_H * (I // 64) * 4)  # 3,342,336 B
FLOPS_PER_SLOT = 2 * (2 * I * H + H * I)  # gate_up + down of one (token, expert) pair


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20, help="steps per timed sample (each config)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--samples", type=int, default=7, help="timed samples; the median is reported")
    ap.add_argument("--layers", type=int, default=8, help="layers in the config-2 / 3 / 4 / 5 rotations")
    ap.add_argument("--only", default="all", help="comma list of: decode, prefill, cfg1, cfg3, cfg5, kernels (or "
                    "hc with --hc: the mix timings alone)")
    ap.add_argument("--hc", action="store_true", help="also time the hyper-connection mix beside the path (logged)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baselines")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--peaks", action="store_true", help="also measure this device's read / copy / MFMA peaks")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run 4 plain 256 MiB device copies (the known-size reference for FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_gate_up_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the decode gate_up kernel, from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarized
    in profiles/ (a line `traffic_bytes_per_launch: N`), or None when that summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip().split()[0])
    except OSError:
        pass
    return None


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Timer:
    """Median over samples of the per-step time of `fn(i)` (i = step index) on the current stream, in ms."""

    def __init__(self, torch, samples: int, steps: int, warmup: int):
        self.torch, self.samples, self.steps, self.warmup = torch, samples, steps, warmup
        self.e0 = torch.cuda.Event(enable_timing=True)
        self.e1 = torch.cuda.Event(enable_timing=True)

    def steps_ms(self, run, steps: int | None = None) -> float:
        """Median over samples of the per-step time when run(k) enqueues k steps at once."""
        n = steps or self.steps
        run(self.warmup)
        res = []
        for _ in range(self.samples):
            self.torch.cuda.synchronize()
            self.e0.record()
            run(n)
            self.e1.record()
            self.torch.cuda.synchronize()
            res.append(self.e0.elapsed_time(self.e1) / n)
        return statistics.median(res)

    def __call__(self, fn, steps: int | None = None) -> float:
        n = steps or self.steps
        for i in range(self.warmup):
            fn(i)
        res = []
        for _ in range(self.samples):
            self.torch.cuda.synchronize()
            self.e0.record()
            for i in range(n):
                fn(i)
            self.e1.record()
            self.torch.cuda.synchronize()
            res.append(self.e0.elapsed_time(self.e1) / n)
        return statistics.median(res)


def hc_section(torch, moe):
    """The hyper-connection mix beside the path (hc_mix_down / hc_mix_up) at the reference's shape: hidden d 2560, rank
    r 320, 4 streams, Q4 and Q8 weights with group size 64, BF16 streams, token counts 1 .. 4096 (synthetic seeded
    weights; W_up read as chunk-major). Logged only: run under rocprofv3 --kernel-trace for the kernels' durations
    (these HIP-event figures include the wrappers' output allocations)."""
    D, R, G = 2560, 320, 64
    for bits in (4, 8):
        wd = moe.QWeight.synth(bits, 3, "gu_q", "gu_s", 0, R + 4, 4 * D, G)
        wu = moe.QWeight.synth(bits, 3, "dn_q", "dn_s", 0, 4 * D, R, G)
        nw = torch.zeros(4 * D, device="cuda")
        for T in (1, 5, 16, 64, 512, 4096):
            x = moe.synth_bf16_normal(3, "x", T, (T, 4 * D), 1.0)
            h, _, inv = moe.hc_mix_down(x, wd, R, True, 1e-6)
            moe.hc_mix_up(h, wu, x, nw, inv)
            torch.cuda.synchronize()
            reps = 20 if T < 4096 else 5
            e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            e[0].record()
            for _ in range(reps):
                moe.hc_mix_down(x, wd, R, True, 1e-6)
            e[1].record()
            for _ in range(reps):
                moe.hc_mix_up(h, wu, x, nw, inv)
            e[2].record()
            torch.cuda.synchronize()
            log(f"hc Q{bits} T={T}: hc_mix_down {e[0].elapsed_time(e[1]) * 1e3 / reps:.1f} us, hc_mix_up "
                f"{e[1].elapsed_time(e[2]) * 1e3 / reps:.1f} us (HIP events around the calls)")


def capture(torch, fn):
    """fn() captured as one HIP graph (after one eager run on a side stream, as capture requires)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def uniq(torch, ids) -> int:
    return int(torch.unique(ids).numel())


def main():
    args = parse()
    ws_env = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or ws_env != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {ws_env}): this build has no "
              "multi-GPU path; DESIGN.md describes how the layer would shard by expert.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from strixite_amd import moe
    from strixite_amd import _lib

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from gpu_util import zipf_bias

    only = set(args.only.split(","))
    want = lambda name: "all" in only or name in only  # noqa: E731
    torch.cuda.set_device(0)
    dev = "cuda"
    timer = Timer(torch, args.samples, args.steps, args.warmup)
    scratch = torch.zeros(64, dtype=torch.float32, device=dev)
    if args.calibrate:
        ca = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        cb = torch.empty_like(ca)
        for _ in range(4):
            cb.copy_(ca)
        torch.cuda.synchronize()
        del ca, cb

    peaks = None
    if args.peaks:
        L = _lib.lib()
        buf = torch.empty(4 << 30, dtype=torch.uint8, device=dev)
        buf2 = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
        st = torch.cuda.current_stream().cuda_stream
        rd = timer(lambda i: L.strix_calib_read_peak(moe._p(buf), buf.numel(), 4096, moe._p(scratch), st), steps=5)
        cp = timer(lambda i: buf2.copy_(buf[: buf2.numel()]), steps=5)
        flops = [0]

        def mf(i):
            flops[0] = L.strix_calib_mfma_peak(256 * 8, 2000, moe._p(scratch), st)
        mm = timer(mf, steps=5)
        peaks = {"read_GBps": round(buf.numel() / (rd / 1e3) / 1e9, 1),
                 "copy_GBps": round(2 * buf2.numel() / (cp / 1e3) / 1e9, 1),
                 "f16_mfma_TFLOPs": round(flops[0] / (mm / 1e3) / 1e12, 1),
                 "how": "4 GiB streaming read (library kernel), 2 GiB device copy (read + write bytes), 2048 blocks x "
                        "4 waves of 4 independent v_mfma_f32_32x32x16_f16 chains"}
        log("measured peaks:", peaks)
        del buf, buf2
        torch.cuda.empty_cache()

    if args.hc:
        hc_section(torch, moe)
        if args.only == "hc":
            return

    ctx = moe.LayerContext()
    nl = args.layers
    t0 = time.time()
    dlayers = [moe.MoeLayer.synth(H, E, K_TOP, I, seed=args.seed, layer=l) for l in range(nl)]
    # the prefill / stack layers: the same weights with Zipf(1.1) router biases drawn per layer
    players = [moe.MoeLayer(H, E, K_TOP, I, L.router, L.gate_up, L.down,
                            torch.from_numpy(zipf_bias(args.seed + l, E, ZIPF_BETA)).to(dev), L.shared_gate_up,
                            L.shared_down) for l, L in enumerate(dlayers)]
    torch.cuda.synchronize()
    log(f"{nl} layers generated on the device in {time.time() - t0:.1f} s, "
        f"{sum(L.weight_bytes for L in dlayers) / 1e9:.2f} GB of weights")
    line = {"metric": METRIC, "value": None, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "samples": args.samples, "ms_per_step": None, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16"}

    # ------------------------------------------------------------------------------------------------ decode (cfg2)
    Md = 16
    xs = [moe.synth_bf16_normal(args.seed, "x", l, (Md, H), 1.0) for l in range(nl)]
    wsd = [L.workspace(Md) for L in dlayers]
    outs = [dlayers[l].forward(xs[l], ws=wsd[l], ctx=ctx) for l in range(nl)]
    torch.cuda.synchronize()
    # graphs of the first n layers of the stack, n = 1 .. L: a sample of K steps replays the whole stack K // L times
    # and then the first K % L layers, so exactly K layer steps run back to back in as few graph launches as possible
    def stack_graphs(layers, run):
        return [capture(torch, lambda n=n: [run(l) for l in range(n)]) for n in range(1, len(layers) + 1)]

    def stack_steps(graphs, k):
        full, rest = divmod(k, len(graphs))
        for _ in range(full):
            graphs[-1].replay()
        if rest:
            graphs[rest - 1].replay()

    dgraphs = stack_graphs(dlayers, lambda l: dlayers[l].forward(xs[l], ws=wsd[l], out=outs[l], ctx=ctx))
    dec_ms = timer.steps_ms(lambda k: stack_steps(dgraphs, k))
    dec_tps = Md / (dec_ms / 1e3)
    un = [uniq(torch, outs[l]["ids"]) for l in range(nl)]
    dec_bytes = statistics.mean(u * (GU_BYTES_PER_EXPERT + DN_BYTES_PER_EXPERT) + SH_BYTES + ROUTER_BYTES + 2 * Md * H * 2
                                for u in un)
    dec_gbs = dec_bytes / (dec_ms / 1e3) / 1e9
    log(f"cfg2 decode: {dec_ms * 1e3:.1f} us/layer, {dec_tps:,.0f} tokens/s, unique experts {statistics.mean(un):.1f}, "
        f"whole-layer algorithmic {dec_gbs:,.0f} GB/s ({dec_gbs / PEAK_HBM_GBS:.1%})")
    line.update({"value": round(dec_tps, 1), "ms_per_step": round(dec_ms, 5)})
    line["math"] = ("decode: bf16 activations, Q4/Q8 codes as exact bf16 integers, bf16 MFMA, per-group scale/min on "
                    "the FP32 accumulator; prefill Q4 experts: the reference's F16 math (x and dequantized weights in "
                    "f16, f16 MFMA, FP32 accumulation); router logits FP32")
    line["data"] = "synthetic (seeded on the device; independent weights per layer)"
    line["config"] = {"workload": "cfg2: decode 16 tokens (2 slots x (1 + 7 MTP)), H3072 E512 top-10 + shared Q8 g64, "
                                  "I512, Q4 g128 routed; 8-layer rotation (HBM-cold) in HIP graphs",
                      "tokens_per_step": Md, "layers_rotated": nl,
                      "unique_experts_mean": round(statistics.mean(un), 1),
                      "layer_algorithmic_bytes": int(dec_bytes), "layer_algorithmic_GBps": round(dec_gbs, 1),
                      "layer_hbm_frac": round(dec_gbs / PEAK_HBM_GBS, 4)}

    # dominant decode kernel: the grouped gate_up + SwiGLU over the layers' own routing, launched alone
    routes = [moe.moe_group_routes(outs[l]["ids"], E)[0] for l in range(nl)]
    hbuf = [torch.empty((Md * K_TOP, I), dtype=torch.bfloat16, device=dev) for _ in range(nl)]
    torch.cuda.synchronize()
    # one graph of the kernel over the 8 layers' routing (its own launches only, no host gap between them); the
    # exact-weight math the layer's decode runs
    ggu = capture(torch, lambda: [moe.experts_gather_grouped_swiglu(xs[l], dlayers[l].gate_up, E, routes[l], Md, K_TOP,
                                                                    h=hbuf[l], math=moe.MOE_MATH_WMMA_BF16)
                                  for l in range(nl)])
    gu_ms = timer(lambda i: ggu.replay(), steps=max(3, args.steps // nl)) / nl
    gu_bytes = statistics.mean(u * GU_BYTES_PER_EXPERT + Md * H * 2 + Md * K_TOP * I * 2 for u in un)
    gu_gbs = gu_bytes / (gu_ms / 1e3) / 1e9
    log(f"decode gate_up kernel: {gu_ms * 1e3:.1f} us/launch, {gu_bytes / 1e6:.1f} MB -> {gu_gbs:,.0f} GB/s "
        f"({gu_gbs / PEAK_HBM_GBS:.1%} of HBM peak)")
    line["roofline"] = {"bound": "hbm", "kernel": "decode_gate_up_lds_kernel (grouped Q4 gate_up + SwiGLU, <= 16 tokens)",
                        "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                        "algorithmic_bytes_per_launch": int(gu_bytes), "us_per_launch": round(gu_ms * 1e3, 3)}
    line["cpu_baseline"] = None
    line["configs"] = {}

    # --------------------------------------------------------------------------------------------- prefill (cfg4)
    Mp = 4096
    if want("prefill") or want("cfg5"):
        xp = [moe.synth_bf16_normal(args.seed, "x", 100 + l, (Mp, H), 1.0) for l in range(nl)]
        wsp = players[0].workspace(Mp)
        pouts = [players[l].forward(xp[l], ws=wsp, ctx=ctx) for l in range(nl)]
        torch.cuda.synchronize()
    if want("prefill"):
        pgraphs = stack_graphs(players, lambda l: players[l].forward(xp[l], ws=wsp, out=pouts[l], ctx=ctx))
        pre_ms = timer.steps_ms(lambda k: stack_steps(pgraphs, k))
        del pgraphs
        slots = Mp * K_TOP
        flops = slots * FLOPS_PER_SLOT + Mp * FLOPS_PER_SLOT + 2 * Mp * (E + 1) * H
        pre_tflops = flops / (pre_ms / 1e3) / 1e12
        cnt = np.bincount(pouts[0]["ids"].cpu().numpy().ravel(), minlength=E)
        proutes = [moe.moe_group_routes(pouts[l]["ids"], E)[0] for l in range(nl)]
        ph = torch.empty((Mp * K_TOP, I), dtype=torch.bfloat16, device=dev)
        gpg = capture(torch, lambda: [moe.experts_gather_grouped_swiglu(xp[l], players[l].gate_up, E, proutes[l], Mp,
                                                                        K_TOP, h=ph) for l in range(nl)])
        pgu_ms = timer(lambda i: gpg.replay(), steps=max(2, args.steps // nl)) / nl
        del gpg
        # the same projection in the exact-weight kind (MoeMath::WmmaBf16: bf16 MFMA over the scaled codes, each
        # group's scale and min applied on the FP32 accumulators), for comparison only
        gpx = capture(torch, lambda: [moe.experts_gather_grouped_swiglu(xp[l], players[l].gate_up, E, proutes[l], Mp,
                                                                        K_TOP, h=ph, math=moe.MOE_MATH_WMMA_BF16)
                                      for l in range(nl)])
        pgx_ms = timer(lambda i: gpx.replay(), steps=max(2, args.steps // nl)) / nl
        del gpx
        pgu_tflops = slots * 2 * 2 * I * H / (pgu_ms / 1e3) / 1e12
        line["prefill"] = {
            "workload": "cfg4: prefill 4096 tokens, Zipf(1.1) router bias (beta 1.0), H3072 E512 top-10 + shared Q8, "
                        "I512, Q4 g128 routed; 8-layer rotation in HIP graphs",
            "tokens_per_s": round(Mp / (pre_ms / 1e3), 1), "ms_per_step": round(pre_ms, 4),
            "layer_flops": flops, "layer_tflops": round(pre_tflops, 2),
            "layer_mfma_frac": round(pre_tflops / PEAK_F16_TFLOPS, 4),
            "roofline": {"bound": "mfma", "kernel": "expert_gemm2_kernel (F16-math grouped Q4 gate_up + SwiGLU)",
                         "achieved": round(pgu_tflops, 2), "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pgu_tflops / PEAK_F16_TFLOPS, 4), "us_per_launch": round(pgu_ms * 1e3, 2),
                         "algorithmic_flops_per_launch": slots * 2 * 2 * I * H},
            "experts_with_0_rows": int((cnt == 0).sum()), "max_rows_per_expert": int(cnt.max()),
            "gate_up_exact_weights_us": round(pgx_ms * 1e3, 2),
        }
        log(f"cfg4 prefill: {pre_ms:.3f} ms/layer, {Mp / (pre_ms / 1e3):,.0f} tokens/s, {pre_tflops:.1f} TFLOP/s "
            f"({pre_tflops / PEAK_F16_TFLOPS:.1%} MFMA); gate_up {pgu_ms * 1e3:.0f} us = {pgu_tflops:.1f} TFLOP/s; "
            f"exact-weight kind {pgx_ms * 1e3:.0f} us")

    # ---------------------------------------------------------------------------------------- cfg1: 1-token Q8 decode
    if want("cfg1"):
        n1 = 24  # 24 x 27 MB of active experts a rotation: far past the MALL
        l1 = [moe.MoeLayer.synth(C1_H, C1_E, C1_K, I, seed=args.seed, layer=l, routed_bits=8, shared=False)
              for l in range(n1)]
        x1 = [moe.synth_bf16_normal(args.seed, "x", 200 + l, (1, C1_H), 1.0) for l in range(n1)]
        w1 = [L.workspace(1) for L in l1]
        o1 = [l1[l].forward(x1[l], ws=w1[l]) for l in range(n1)]
        torch.cuda.synchronize()
        g1 = stack_graphs(l1, lambda l: l1[l].forward(x1[l], ws=w1[l], out=o1[l]))
        ms1 = timer.steps_ms(lambda k: stack_steps(g1, k))
        b1 = statistics.mean(uniq(torch, o1[l]["ids"]) * C1_BYTES_PER_EXPERT + C1_E * C1_H * 2 + 2 * C1_H * 2
                             for l in range(n1))
        line["configs"]["cfg1"] = {
            "workload": "cfg1: decode 1 token, H2048 E64 top-8, I512, Q8 g64 routed, no shared; 24-layer rotation",
            "tokens_per_s": round(1 / (ms1 / 1e3), 1), "us_per_step": round(ms1 * 1e3, 2),
            "algorithmic_bytes": int(b1), "GBps": round(b1 / (ms1 / 1e3) / 1e9, 1),
            "hbm_frac": round(b1 / (ms1 / 1e3) / 1e9 / PEAK_HBM_GBS, 4)}
        log("cfg1:", line["configs"]["cfg1"])
        del g1, l1, x1, w1, o1
        torch.cuda.empty_cache()

    # --------------------------------------------------------------------------- cfg3: 512-token uniform-logit prefill
    if want("cfg3"):
        M3 = 512
        x3 = [moe.synth_bf16_normal(args.seed, "x", 300 + l, (M3, H), 1.0) for l in range(nl)]
        lg3 = [moe.synth_uniform_pm1(args.seed, "logits", l, (M3, E + 1)) for l in range(nl)]
        w3 = dlayers[0].workspace(M3)
        o3 = [dlayers[l].forward(x3[l], logits_in=lg3[l], ws=w3, ctx=ctx) for l in range(nl)]
        torch.cuda.synchronize()
        g3 = stack_graphs(dlayers, lambda l: dlayers[l].forward(x3[l], logits_in=lg3[l], ws=w3, out=o3[l], ctx=ctx))
        ms3 = timer.steps_ms(lambda k: stack_steps(g3, k))
        u3 = statistics.mean(uniq(torch, o3[l]["ids"]) for l in range(nl))
        b3 = u3 * (GU_BYTES_PER_EXPERT + DN_BYTES_PER_EXPERT) + SH_BYTES + 2 * M3 * H * 2
        f3 = M3 * K_TOP * FLOPS_PER_SLOT + M3 * FLOPS_PER_SLOT
        line["configs"]["cfg3"] = {
            "workload": "cfg3: prefill 512 tokens, router bypassed with uniform logits U(-1, 1), H3072 E512 top-10 + "
                        "shared Q8, I512, Q4 g128; 8-layer rotation",
            "tokens_per_s": round(M3 / (ms3 / 1e3), 1), "us_per_step": round(ms3 * 1e3, 2),
            "unique_experts_mean": round(u3, 1), "algorithmic_bytes": int(b3),
            "GBps": round(b3 / (ms3 / 1e3) / 1e9, 1), "hbm_frac": round(b3 / (ms3 / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
            "TFLOPs": round(f3 / (ms3 / 1e3) / 1e12, 2)}
        log("cfg3:", line["configs"]["cfg3"])
        del g3

    # ------------------------------------------------------ cfg5: an 8-layer stack, decode 16 then prefill 4096 tokens
    if want("cfg5"):
        x5d = [moe.synth_bf16_normal(args.seed, "x", 500 + l, (Md, H), 1.0) for l in range(nl)]
        w5d = players[0].workspace(Md)
        o5d = [players[l].forward(x5d[l], ws=w5d, ctx=ctx) for l in range(nl)]
        torch.cuda.synchronize()

        def stack():
            for l in range(nl):
                players[l].forward(x5d[l], ws=w5d, out=o5d[l], ctx=ctx)
            for l in range(nl):
                players[l].forward(xp[l], ws=wsp, out=pouts[l], ctx=ctx)
        g5 = capture(torch, stack)
        ms5 = timer(lambda i: g5.replay(), steps=max(2, args.steps // 4))
        u5 = statistics.mean(uniq(torch, o5d[l]["ids"]) for l in range(nl))
        b5 = nl * (u5 * (GU_BYTES_PER_EXPERT + DN_BYTES_PER_EXPERT) + SH_BYTES + ROUTER_BYTES + 2 * Md * H * 2)
        f5 = nl * (Mp * K_TOP * FLOPS_PER_SLOT + Mp * FLOPS_PER_SLOT + 2 * Mp * (E + 1) * H)
        line["configs"]["cfg5"] = {
            "workload": "cfg5: 8-layer stack (independent weights, Zipf router biases per layer), a 16-token decode step "
                        "then a 4096-token prefill step through all 8 layers, one HIP graph",
            "ms_per_stack_step": round(ms5, 4), "tokens_per_s": round((Md + Mp) / (ms5 / 1e3), 1),
            "decode_bytes": int(b5), "prefill_flops": f5}
        log("cfg5:", line["configs"]["cfg5"])
        del g5

    # --------------------------------------------------------------------------------------------- CPU baselines
    if not args.no_cpu:
        import oracle as orc
        from gpu_util import oracle_weights, to_np

        threads = args.cpu_threads or max(1, min(16, len(os.sched_getaffinity(0))))

        def cpu_time(fn, budget_s):
            fn()  # warm
            times = []
            t_end = time.time() + budget_s
            while len(times) < 7 and (len(times) < 3 or time.time() < t_end):
                t1 = time.perf_counter()
                fn()
                times.append(time.perf_counter() - t1)
            return statistics.median(times), len(times)

        w0 = oracle_weights(dlayers[0])
        x0 = to_np(xs[0])
        cpu_s, n = cpu_time(lambda: orc.moe_layer(w0, x0, threads=threads), 10.0)
        line["cpu_baseline"] = {
            "value": round(Md / cpu_s, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle/ C restatement, the full cfg2 layer (16 tokens, layer 0 weights), median of {n} runs "
                      f"({cpu_s * 1e3:.1f} ms each); host nproc {os.cpu_count()}"}
        log(f"cpu oracle cfg2: {cpu_s * 1e3:.1f} ms/layer on {threads} threads -> {Md / cpu_s:.1f} tokens/s")
        if want("prefill"):
            Ms = 64
            wp = oracle_weights(players[0])
            xs4 = np.ascontiguousarray(to_np(xp[0])[:Ms])
            cpu4, n4 = cpu_time(lambda: orc.moe_layer(wp, xs4, threads=threads), 10.0)
            line["prefill"]["cpu_baseline"] = {
                "value": round(Ms / cpu4, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"oracle/ C restatement, the cfg4 layer (layer 0 weights and Zipf bias) on the first {Ms} of "
                          f"the 4096 tokens, median of {n4} runs ({cpu4 * 1e3:.1f} ms each)"}
            log(f"cpu oracle cfg4 sample: {cpu4 * 1e3:.1f} ms for {Ms} tokens -> {Ms / cpu4:.1f} tokens/s")

    if peaks is not None:
        line["peaks_measured"] = peaks
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
