"""Benchmark of the MoE FFN sublayer on one MI355X: BASELINE config 2 (16-token decode step, the headline `value`)
and config 4 (4096-token Zipf prefill), each over an 8-layer stack of independent weights (~10.3 GB, so every step
reads its experts from HBM, not the 256 MB MALL). Prints ONE JSON line.

A step is one MoE sublayer forward (router projection -> top-k -> packing -> gate_up + SwiGLU -> down -> ordered
combine + shared expert -> residual) over one batch, layer l = step % 8; the 8 layer steps are captured as one HIP
graph, replayed whole (a decode step through the stack). Inputs are resident in HBM before the timed region. The dominant kernel's duration is measured separately with HIP events on the launch stream and converted to
a roofline fraction; the CPU oracle (multithreaded C) is timed on the host beside it.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tokens/s; achieved HBM GB/s (decode) and MFMA % of peak (prefill)"
PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # dense fp16/bf16 MFMA

H, E, K_TOP, I = 3072, 512, 10, 512
GU_BYTES_PER_EXPERT = 2 * I * H // 2 + 2 * I * (H // 128) * 4    # Q4 g128 gate_up: 1,671,168 B
DN_BYTES_PER_EXPERT = H * I // 2 + H * (I // 128) * 4            # Q4 g128 down: 835,584 B
SH_BYTES = 2 * I * H + 2 * I * (H // 64) * 4 + H * I + H * (I // 64) * 4  # Q8 g64 shared: 5,013,504 B
ROUTER_BYTES = (E + 1) * H * 2
ZIPF_BETA = 1.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--prefill-steps", type=int, default=24)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of one HIP graph per layer")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--seed", type=int, default=0)
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


def main():
    args = parse()
    ws_env = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or ws_env != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {ws_env}): this build has no "
              "multi-GPU path; see DESIGN.md for how the layer would shard by expert.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from strixite_amd import moe

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from gpu_util import zipf_bias

    torch.cuda.set_device(0)
    dev = "cuda"
    if args.calibrate:
        ca = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        cb = torch.empty_like(ca)
        for _ in range(4):
            cb.copy_(ca)
        torch.cuda.synchronize()
        del ca, cb
    nl = args.layers
    t0 = time.time()
    layers = []
    for l in range(nl):
        bias = torch.from_numpy(zipf_bias(args.seed + l, E, ZIPF_BETA)).to(dev)
        layers.append(moe.MoeLayer.synth(H, E, K_TOP, I, seed=args.seed, layer=l, router_bias=None))
        layers[-1]._zipf_bias = bias
    torch.cuda.synchronize()
    log(f"{nl} layers generated on the device in {time.time() - t0:.1f} s, "
        f"{sum(L.weight_bytes for L in layers) / 1e9:.2f} GB of weights")

    # ---------------------------------------------------------------------------------------------- decode (cfg2)
    Md = 16
    xs = [moe.synth_bf16_normal(args.seed, "x", l, (Md, H), 1.0) for l in range(nl)]
    wsd = [L.workspace(Md) for L in layers]
    outs = [None] * nl
    for l in range(nl):
        outs[l] = layers[l].forward(xs[l], ws=wsd[l])
    torch.cuda.synchronize()

    def run_layer(l):
        layers[l].forward(xs[l], ws=wsd[l], out=outs[l])

    # One HIP graph holds the whole 8-layer stack (one decode step through the stack, as an engine captures its
    # forward): a replay runs 8 layer steps, so per-launch overhead is paid once per stack, not once per layer.
    graph = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for l in range(nl):
                run_layer(l)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for l in range(nl):
                run_layer(l)
        torch.cuda.synchronize()

    def run_steps(n):
        """n layer steps (whole stacks: n is rounded up to a multiple of the layer count); returns the steps run"""
        stacks = (n + nl - 1) // nl
        for _ in range(stacks):
            if graph is not None:
                graph.replay()
            else:
                for l in range(nl):
                    run_layer(l)
        return stacks * nl

    run_steps(args.warmup)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    steps_run = run_steps(args.steps)
    ev1.record()
    torch.cuda.synchronize()
    dec_ms = ev0.elapsed_time(ev1) / steps_run
    dec_tps = Md / (dec_ms / 1e3)
    uniq = [len(np.unique(outs[l]["ids"].cpu().numpy())) for l in range(nl)]
    dec_bytes = [u * (GU_BYTES_PER_EXPERT + DN_BYTES_PER_EXPERT) + SH_BYTES + ROUTER_BYTES + 2 * Md * H * 2
                 for u in uniq]
    dec_layer_gbs = statistics.mean(dec_bytes) / (dec_ms / 1e3) / 1e9
    log(f"decode: {dec_ms * 1e3:.1f} us/layer, {dec_tps:,.0f} tokens/s, unique experts {statistics.mean(uniq):.1f}, "
        f"whole-layer algorithmic {dec_layer_gbs:,.0f} GB/s")

    # dominant decode kernel: the grouped gate_up + SwiGLU over the layer's own routing, timed alone
    routes = [moe.moe_group_routes(outs[l]["ids"], E)[0] for l in range(nl)]
    hbuf = [torch.empty((Md * K_TOP, I), dtype=torch.bfloat16, device=dev) for _ in range(nl)]
    torch.cuda.synchronize()

    def gu_launch(l):
        moe.experts_gather_grouped_swiglu(xs[l], layers[l].gate_up, E, routes[l], Md, K_TOP, h=hbuf[l])

    for i in range(args.warmup):
        gu_launch(i % nl)
    torch.cuda.synchronize()
    reps = max(args.steps, 8 * nl)
    ev0.record()
    for i in range(reps):
        gu_launch(i % nl)
    ev1.record()
    torch.cuda.synchronize()
    gu_us = ev0.elapsed_time(ev1) / reps * 1e3
    gu_bytes = statistics.mean(u * GU_BYTES_PER_EXPERT + Md * H * 2 + Md * K_TOP * I * 2 for u in uniq)
    gu_gbs = gu_bytes / (gu_us / 1e6) / 1e9
    log(f"decode gate_up kernel: {gu_us:.1f} us/launch, {gu_bytes / 1e6:.1f} MB -> {gu_gbs:,.0f} GB/s "
        f"({gu_gbs / PEAK_HBM_GBS:.1%} of HBM peak)")

    # --------------------------------------------------------------------------------------------- prefill (cfg4)
    Mp = 4096
    pre = {}
    if args.prefill_steps > 0:
        xp = moe.synth_bf16_normal(args.seed, "x", 100, (Mp, H), 1.0)
        players = [moe.MoeLayer(H, E, K_TOP, I, L.router, L.gate_up, L.down, L._zipf_bias, L.shared_gate_up,
                                L.shared_down) for L in layers]
        wsp = players[0].workspace(Mp)
        pouts = [players[l].forward(xp, ws=wsp) for l in range(nl)]
        torch.cuda.synchronize()
        for i in range(2):
            players[i % nl].forward(xp, ws=wsp, out=pouts[i % nl])
        torch.cuda.synchronize()
        ev0.record()
        for i in range(args.prefill_steps):
            players[i % nl].forward(xp, ws=wsp, out=pouts[i % nl])
        ev1.record()
        torch.cuda.synchronize()
        pre_ms = ev0.elapsed_time(ev1) / args.prefill_steps
        flops = 2 * Mp * K_TOP * (2 * I * H + H * I) + 2 * Mp * (2 * I * H + H * I) + 2 * Mp * (E + 1) * H
        pre_tflops = flops / (pre_ms / 1e3) / 1e12
        cnt = np.bincount(pouts[0]["ids"].cpu().numpy().ravel(), minlength=E)
        # dominant prefill kernel: the grouped gate_up + SwiGLU
        proutes = [moe.moe_group_routes(pouts[l]["ids"], E)[0] for l in range(nl)]
        ph = torch.empty((Mp * K_TOP, I), dtype=torch.bfloat16, device=dev)
        moe.experts_gather_grouped_swiglu(xp, players[0].gate_up, E, proutes[0], Mp, K_TOP, h=ph)
        torch.cuda.synchronize()
        preps = 2 * nl
        ev0.record()
        for i in range(preps):
            moe.experts_gather_grouped_swiglu(xp, players[i % nl].gate_up, E, proutes[i % nl], Mp, K_TOP, h=ph)
        ev1.record()
        torch.cuda.synchronize()
        pgu_us = ev0.elapsed_time(ev1) / preps * 1e3
        pgu_flops = 2 * Mp * K_TOP * 2 * I * H
        pgu_tflops = pgu_flops / (pgu_us / 1e6) / 1e12
        pre = {
            "workload": "cfg4: prefill 4096 tokens, Zipf(1.1) router bias (beta 1.0), H3072 E512 top-10 + shared Q8, "
                        "I512, Q4 g128 routed",
            "tokens_per_s": round(Mp / (pre_ms / 1e3), 1), "ms_per_step": round(pre_ms, 4),
            "layer_tflops": round(pre_tflops, 2), "layer_mfma_frac": round(pre_tflops / PEAK_F16_TFLOPS, 4),
            "gate_up_kernel": {"us": round(pgu_us, 2), "tflops": round(pgu_tflops, 2),
                               "mfma_frac": round(pgu_tflops / PEAK_F16_TFLOPS, 4)},
            "experts_with_0_rows": int((cnt == 0).sum()), "max_rows_per_expert": int(cnt.max()),
            "steps": args.prefill_steps,
        }
        log(f"prefill: {pre_ms:.3f} ms/layer, {Mp / (pre_ms / 1e3):,.0f} tokens/s, {pre_tflops:.1f} TFLOP/s "
            f"({pre_tflops / PEAK_F16_TFLOPS:.1%} MFMA), gate_up {pgu_us:.0f} us = {pgu_tflops:.1f} TFLOP/s")

    # ------------------------------------------------------------------------------------------- CPU baseline (cfg2)
    cpu = None
    if not args.no_cpu:
        import oracle as orc
        from gpu_util import oracle_weights, to_np

        threads = args.cpu_threads or max(1, min(16, len(os.sched_getaffinity(0))))
        w0 = oracle_weights(layers[0])
        x0 = to_np(xs[0])
        orc.moe_layer(w0, x0, threads=threads)  # warm
        times = []
        t_end = time.time() + 10.0
        while len(times) < 7 and (len(times) < 3 or time.time() < t_end):
            t1 = time.perf_counter()
            orc.moe_layer(w0, x0, threads=threads)
            times.append(time.perf_counter() - t1)
        cpu_s = statistics.median(times)
        cpu = {"value": round(Md / cpu_s, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
               "sample": f"oracle/ C restatement, full cfg2 layer (16 tokens, layer 0 weights), median of {len(times)} "
                         f"runs ({cpu_s * 1e3:.1f} ms each); host nproc {os.cpu_count()}"}
        log(f"cpu oracle: {cpu_s * 1e3:.1f} ms/layer on {threads} threads -> {Md / cpu_s:.1f} tokens/s")

    line = {
        "metric": METRIC, "value": round(dec_tps, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps_run,
        "warmup": args.warmup, "ms_per_step": round(dec_ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "math": "decode: bf16 activations, Q4/Q8 codes as exact bf16 integers, bf16 MFMA, per-group scale/min on the FP32 "
                "accumulator; prefill Q4 experts: the reference's F16 math (x and dequantized weights in f16, f16 MFMA, "
                "FP32 accumulation); router logits FP32",
        "data": "synthetic (seeded on the device; independent weights per layer)",
        "config": {"workload": "cfg2: decode 16 tokens (2 slots x (1 + 7 MTP)), H3072 E512 top-10 + shared Q8 g64, "
                               "I512, Q4 g128 routed; 8-layer stack rotated (HBM-cold)",
                   "tokens_per_step": Md, "layers_rotated": nl, "graph": "one HIP graph per 8-layer stack" if graph is not None else None,
                   "unique_experts_mean": round(statistics.mean(uniq), 1),
                   "layer_algorithmic_GBps": round(dec_layer_gbs, 1)},
        "roofline": {"bound": "hbm", "kernel": "expert_stream_kernel<Q4, GROUPED, SWIGLU> (decode gate_up + SwiGLU)",
                     "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                     "algorithmic_bytes_per_launch": int(gu_bytes), "us_per_launch": round(gu_us, 3)},
        "cpu_baseline": cpu,
        "prefill": pre,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
