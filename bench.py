"""MoE layer throughput on one MI355X: the 35B-A3B-shaped W4A16 layer (T=2048 tokens, H=2048, 256 experts top-8,
I=512, shared expert 512, int4 group-128 weights), one step = one full layer forward (router, routed experts,
gated shared expert, combine) through the HIP path.

    python bench.py [--steps K] [--warmup W] [--config headline] [--no-cpu] [--eager]

Timing: W untimed forwards, then K forwards replayed from one HIP graph capture of the layer (the way the reference
serves, a level per graph), bracketed by device synchronisation. Inputs and weights are resident in HBM before the
timed region. Separately, an eager pass with stage events (the library's profiling hook) times each kernel stage;
the dominant kernel's average duration gives the roofline entry. The CPU baseline is the reference's CPU algorithm
(dequantise-per-call + padded bmm, oracle/cpu_bmm.py) on the same inputs, on all host cores, on a bounded sample.
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np
import torch

METRIC = "MoE layer tokens/s at T=2048 (35B-A3B shape); % of HBM/MFMA roofline"
HBM_PEAK = 8.0e12        # bytes/s, MI355X
MFMA_BF16_PEAK = 2.5e15  # dense bf16 FLOP/s, MI355X


def layer_work(cfg, idx: np.ndarray) -> dict:
    """Algorithmic work of one layer forward and of its gate_up launch, from the realised routing."""
    T, H, E, k, I, I_s = cfg.T, cfg.H, cfg.E, cfg.k, cfg.I, cfg.I_s
    n_hit = int(np.count_nonzero(np.bincount(idx.reshape(-1), minlength=E)))
    A = T * k
    b_gu = 2 * I * H // 2 + 2 * I * (H // 128) * 2          # gate_up words + scales, one expert
    b_dn = H * I // 2 + H * (I // 128) * 2
    b_sgu = 2 * I_s * H // 2 + 2 * I_s * (H // 128) * 2
    b_sdn = H * I_s // 2 + H * (I_s // 128) * 2
    flops = T * (2 * E * H + 6 * k * I * H + 6 * I_s * H + 2 * H)
    layer_bytes = n_hit * (b_gu + b_dn) + b_sgu + b_sdn + (H * 2 if I_s else 0) + E * H * 4 + 2 * T * H * 2
    gu_bytes = n_hit * b_gu + b_sgu + T * H * 2 + (A * I + T * I_s) * 2   # weights, x read, h written
    gu_flops = 2 * A * H * 2 * I + 2 * T * H * 2 * I_s
    return dict(n_hit=n_hit, flops=flops, bytes=layer_bytes, gu_bytes=gu_bytes, gu_flops=gu_flops)


def cpu_baseline(layer, x, k, budget_s: float = 30.0) -> dict:
    from oracle import cpu_bmm

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    lay = {n: (None if t is None else t.cpu()) for n, t in layer.items()}
    xc = x.cpu()
    t0 = time.perf_counter()
    cpu_bmm.layer_forward(lay, xc, k)          # warm-up
    first = time.perf_counter() - t0
    calls = max(1, min(3, int(budget_s / max(first, 1e-3)) - 1))
    times = []
    for _ in range(calls):
        t0 = time.perf_counter()
        cpu_bmm.layer_forward(lay, xc, k)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    return {"value": x.shape[0] / t, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"full layer at T={x.shape[0]}: median of {calls} calls after 1 warm-up "
                      f"({t:.2f} s per call, torch CPU, {platform.processor() or platform.machine()})"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="headline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of graph replay")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (counter calibration) and exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this MoE layer runs on a single MI355X by design (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE {world}); run it with --gpus 1", file=sys.stderr)
        return 2

    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 5}))
        return 0

    from janus_amd import _lib, synth
    from janus_amd.block import W4A16SparseMoeBlock

    cfg = synth.CONFIGS[args.config]
    layer = synth.layer(cfg)
    x = synth.activations(cfg).to(dev)
    blk = W4A16SparseMoeBlock.from_tensors(layer, cfg.k).to(dev)
    with torch.no_grad():
        out = blk(x)                            # router prep, first launch
        _, _, idx = blk.gate(x)
    torch.cuda.synchronize()
    work = layer_work(cfg, idx.cpu().numpy())

    def step():
        with torch.no_grad():
            return blk(x)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    graph = None
    if not args.eager:
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = step()
        for _ in range(3):
            graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        if graph is not None:
            graph.replay()
        else:
            step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3

    # stage timing with events on the launch stream (eager)
    L = _lib.lib()
    names = ("route", "align", "gate_up", "down", "finalize")
    sums = np.zeros(len(names))
    reps = max(5, min(args.steps, 50))
    for _ in range(reps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        for e in ev:
            e.record()                          # creates the underlying hipEvent
        handles = (ctypes.c_void_p * 6)(*[ctypes.c_void_p(e.cuda_event) for e in ev])
        L.janus_moe_profile_events(handles, 6)
        step()
        L.janus_moe_profile_events(None, 0)
        torch.cuda.synchronize()
        sums += [ev[i].elapsed_time(ev[i + 1]) for i in range(5)]
    stage_us = {n: float(v / reps * 1e3) for n, v in zip(names, sums)}

    gu_s = stage_us["gate_up"] * 1e-6
    t_step = ms * 1e-3
    t_roof = max(work["flops"] / MFMA_BF16_PEAK, work["bytes"] / HBM_PEAK)
    gu_bound_hbm = work["gu_bytes"] / HBM_PEAK >= work["gu_flops"] / MFMA_BF16_PEAK
    if gu_bound_hbm:
        ach = work["gu_bytes"] / gu_s / 1e9
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": ach / (HBM_PEAK / 1e9)}
    else:
        ach = work["gu_flops"] / gu_s / 1e12
        roof = {"bound": "mfma", "achieved": ach, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": ach / (MFMA_BF16_PEAK / 1e12)}
    roof.update({"kernel": "w4a16_gemm_kernel<gate_up>", "algorithmic_bytes": work["gu_bytes"],
                 "algorithmic_flops": work["gu_flops"], "avg_us": stage_us["gate_up"], "traffic": None})

    result = {
        "metric": METRIC, "value": cfg.T / t_step, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: seeded splitmix64 activations and random int4 g128 weights",
        "config": {"workload": f"W4A16 MoE layer {cfg.name}: T={cfg.T} H={cfg.H} E={cfg.E} top{cfg.k} I={cfg.I} "
                               f"shared I={cfg.I_s}", "T": cfg.T, "H": cfg.H, "experts": cfg.E, "top_k": cfg.k,
                   "I": cfg.I, "I_shared": cfg.I_s, "codec": "int4 group-128, bf16 scales",
                   "timing": "eager launches" if graph is None else "HIP graph replay"},
        "roofline": roof,
        "layer_roofline": {"t_roof_us": t_roof * 1e6, "t_us": t_step * 1e6, "frac": t_roof / t_step,
                           "bound": "hbm" if work["bytes"] / HBM_PEAK >= work["flops"] / MFMA_BF16_PEAK else "mfma",
                           "flops": work["flops"], "bytes": work["bytes"], "n_hit": work["n_hit"]},
        "stages_us": stage_us,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(layer, x, cfg.k)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
