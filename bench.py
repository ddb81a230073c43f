"""MoE layer throughput on one MI355X: the 35B-A3B-shaped W4A16 layer (T=2048 tokens, H=2048, 256 experts top-8,
I=512, shared expert 512, int4 group-128 weights), one step = one full layer forward (router, routed experts,
gated shared expert, combine) through the HIP path.

    python bench.py [--steps K] [--warmup W] [--config headline] [--no-cpu] [--no-pmc] [--gpus 1]

Timed region: W untimed forwards, then K forwards launched back to back on one stream, bracketed by device
synchronisation. Inputs and weights are resident in HBM before it starts. The stage breakdown comes from K more
forwards in which the library records HIP events on its launch stream at the stage boundaries
(janus_moe_profile_events), each step into its own events; each event is a command-processor packet between two
kernels (a few us each, measured), so those steps are not the timed ones. The dominant kernel (both grouped GEMMs, gate_up and down,
in one persistent launch) gives the roofline entry; its HBM traffic per launch comes from two rocprofv3 --pmc child
runs of this script (FETCH_SIZE, then WRITE_SIZE), each scaled by what the same counter reads for a device copy of
known size. With JANUS_MOE_SCHEDULE=split in the environment the GEMMs run as one launch each (the A/B reference):
the stages then also report gate_up and down, and the traffic entry is null. The same layer replayed
from a HIP graph is timed afterwards and reported as graph_tokens_per_s. The CPU baseline is the reference's CPU
algorithm (dequantise-per-call + padded bmm, oracle/cpu_bmm.py) on the same inputs, on all host cores, on a bounded
sample. `variants_us` times the paths beside the headline one on the same inputs (right-padding mask, the serving
sequence fused and unfused, NVFP4 stacks). Prints one JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import re
import json
import os
import platform
import sqlite3
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np
import torch

METRIC = "MoE layer tokens/s at T=2048 (35B-A3B shape); % of HBM/MFMA roofline"
HBM_PEAK = 8.0e12        # bytes/s, MI355X
MFMA_BF16_PEAK = 2.5e15  # dense bf16 FLOP/s, MI355X
STAGES = ("route", "align", "gate_up", "down", "combine")  # the library's event boundaries
EXPERTS_KERNEL = r"moe_experts_kernel<"      # gate_up + down in one persistent launch
COPY_MIB = 256
HERE = Path(__file__).resolve().parent


def layer_work(cfg, idx: np.ndarray) -> dict:
    """Algorithmic work of one layer forward and of its expert GEMMs (gate_up + down, routed + shared), from the
    realised routing. The intermediate h is not algorithmic; the GEMMs' algorithmic output is the [T, H] bf16 sum."""
    T, H, E, k, I, I_s = cfg.T, cfg.H, cfg.E, cfg.k, cfg.I, cfg.I_s
    n_hit = int(np.count_nonzero(np.bincount(idx.reshape(-1), minlength=E)))
    A = T * k
    b_gu = 2 * I * H // 2 + 2 * I * (H // 128) * 2          # gate_up words + scales, one expert
    b_dn = H * I // 2 + H * (I // 128) * 2
    b_sgu = 2 * I_s * H // 2 + 2 * I_s * (H // 128) * 2
    b_sdn = H * I_s // 2 + H * (I_s // 128) * 2
    flops = T * (2 * E * H + 6 * k * I * H + 6 * I_s * H + 2 * H)
    layer_bytes = n_hit * (b_gu + b_dn) + b_sgu + b_sdn + (H * 2 if I_s else 0) + E * H * 4 + 2 * T * H * 2
    ex_bytes = n_hit * (b_gu + b_dn) + b_sgu + b_sdn + 2 * T * H * 2            # weights, x read, output written
    ex_flops = 6 * A * I * H + 6 * T * I_s * H
    return dict(n_hit=n_hit, flops=flops, bytes=layer_bytes, ex_bytes=ex_bytes, ex_flops=ex_flops)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else what platform reports."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def rel_l2(a, b) -> float:
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def cpu_baseline(layer, x, k, gpu_out: torch.Tensor, budget_s: float = 30.0, n_check: int = 16) -> dict:
    """The reference's CPU algorithm timed on the host cores, and checked in the same run: its output on the first
    n_check tokens against the oracle's, and on every token against the HIP path's output."""
    from oracle import cpu_bmm, oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    lay = {n: (None if t is None else t.cpu()) for n, t in layer.items()}
    xc = x.cpu()
    t0 = time.perf_counter()
    out = cpu_bmm.layer_forward(lay, xc, k)    # warm-up, and the output checked below
    first = time.perf_counter() - t0
    calls = max(1, min(3, int(budget_s / max(first, 1e-3)) - 1))
    times = []
    for _ in range(calls):
        t0 = time.perf_counter()
        cpu_bmm.layer_forward(lay, xc, k)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    tokens = np.arange(min(n_check, x.shape[0]))
    want = oracle.block_forward(oracle.numpy_layer(lay), oracle.bf16_values(xc), k, tokens=tokens)[0]
    check = {"tokens_vs_oracle": int(tokens.size), "rel_l2_vs_oracle": rel_l2(out[tokens].float().numpy(), want),
             "rel_l2_vs_hip": rel_l2(out.float().numpy(), gpu_out.float().cpu().numpy())}
    return {"value": x.shape[0] / t, "unit": "tokens/s", "cores": cores, "kind": "port", "cpu": cpu_model(),
            "sample": f"full layer at T={x.shape[0]}: median of {calls} calls after 1 warm-up "
                      f"({t:.2f} s per call, torch CPU on {cores} threads)", "check": check}


def make_layer(name: str, dev: torch.device):
    from janus_amd import synth
    from janus_amd.block import W4A16SparseMoeBlock

    cfg = synth.CONFIGS[name]
    layer = synth.layer(cfg)
    x = synth.activations(cfg).to(dev)
    blk = W4A16SparseMoeBlock.from_tensors(layer, cfg.k).to(dev)
    return cfg, layer, x, blk


# ---- the paths beside the headline one -------------------------------------------------------------------------

def _time_us(fn, iters: int = 20) -> float:
    """Average device time of fn() over `iters` eager calls after 3 warm-ups, HIP events on the current stream."""
    for _ in range(3):
        fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / iters


class _Norm(torch.nn.Module):
    """A Qwen3_5RMSNorm's two attributes (weight, eps), for the serving sequence."""

    def __init__(self, weight, eps=1e-6):
        super().__init__()
        self.weight, self.eps = weight, eps


def variant_timings(cfg, x, blk, dev, rounds: int = 3) -> dict:
    """Device time per call (us) of the paths beside the headline layer, on the same inputs:
      - layer: the headline layer itself, measured in the same rounds as the others (the reference point);
      - masked_25pct: the layer with a level batch's right padding (8 rows, a quarter of the positions padding);
      - serve_unfused / serve_fused: _add_norm, the layer and the next _add_norm as three calls, and as one call whose
        combine writes the second _add_norm;
      - experts_int4 / experts_nvfp4: fused_moe on the layer's routing with the int4 stacks and with NVFP4 stacks of
        the same shape (random weights quantised on the GPU);
      - block_nvfp4: the whole layer (router, routed and shared experts) with the same layer's weights re-encoded in
        NVFP4 (synth.nvfp4_layer, quantised on the GPU), one block_forward_nvfp4 call.
    The paths are timed in `rounds` interleaved rounds and each reports its median, so a clock or box drift during
    the measurement moves them together. Each entry that fails is reported as its error text instead."""
    from janus_amd import ops, synth
    from janus_amd.block import NVFP4SparseMoeBlock
    from janus_amd.hybrid import nvfp4_quantize
    from janus_amd.moe_w4a16 import fused_moe

    out, cases = {}, {}
    g = torch.Generator(device=dev).manual_seed(5)
    cases["layer"] = lambda: blk(x)

    rows = 8
    length = cfg.T // rows
    lengths = torch.full((rows,), length, device=dev)
    lengths[::2] = length // 2                       # half the rows half full: a quarter of the positions padding
    valid = (torch.arange(length, device=dev)[None] < lengths[:, None]).reshape(-1)
    cases["masked_25pct"] = lambda: blk(x, valid=valid)

    h_attn = (torch.randn(x.shape, generator=g, device=dev) * 0.5).bfloat16()
    post = _Norm((torch.randn(cfg.H, generator=g, device=dev) * 0.1).bfloat16())
    nxt = _Norm((torch.randn(cfg.H, generator=g, device=dev) * 0.1).bfloat16())

    def unfused():
        x1, n1 = ops.add_rmsnorm(x, h_attn, post.weight, post.eps)
        return ops.add_rmsnorm(x1, blk(n1), nxt.weight, nxt.eps)

    cases["serve_unfused"] = unfused
    cases["serve_fused"] = lambda: blk.serve(x, h_attn, post, nxt)

    with torch.no_grad():
        _, w, idx = blk.gate(x)
    ex = blk.experts
    cases["experts_int4"] = lambda: fused_moe(x, idx, w, ex.gate_up, ex.gate_up_scale, None, ex.down, ex.down_scale,
                                              None)
    try:
        def stack(rows_, k):
            parts = [nvfp4_quantize(torch.randn(rows_, k, generator=g, device=dev) * 0.05) for _ in range(cfg.E)]
            return (torch.stack([p[0] for p in parts]), torch.stack([p[1] for p in parts]),
                    torch.stack([p[2] for p in parts])[:, None, None].expand(cfg.E, rows_, 1).contiguous())
        nv_stacks = (*stack(2 * cfg.I, cfg.H), *stack(cfg.H, cfg.I))
        cases["experts_nvfp4"] = lambda: fused_moe(x, idx, w, *nv_stacks)
    except Exception as exc:
        out["experts_nvfp4"] = f"{type(exc).__name__}: {exc}"[:200]
    try:
        nv = NVFP4SparseMoeBlock.from_tensors(synth.nvfp4_layer(cfg, device=dev), cfg.k)
        cases["block_nvfp4"] = lambda: nv(x)
    except Exception as exc:
        out["block_nvfp4"] = f"{type(exc).__name__}: {exc}"[:200]

    times = {name: [] for name in cases}
    for _ in range(rounds):
        for name, fn in cases.items():
            if name in out:
                continue
            try:
                with torch.no_grad():
                    times[name].append(_time_us(fn))
            except Exception as exc:  # an extra line of evidence must not take the headline measurement with it
                out[name] = f"{type(exc).__name__}: {exc}"[:200]
    for name, ts in times.items():
        if name not in out:
            out[name] = float(np.median(ts))
    return out


# ---- counters (child runs under rocprofv3) ---------------------------------------------------------------------

def _pmc_child(args) -> int:
    """What the profiled child runs: a few eager layer forwards, or one device copy of COPY_MIB MiB."""
    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        return 0
    _, _, x, blk = make_layer(args.config, dev)
    with torch.no_grad():
        for _ in range(4):
            blk(x)
    torch.cuda.synchronize()
    return 0


def _counters_per_dispatch(db: Path, counters: list[str], kernel_substr: str) -> dict:
    """Per counter: (mean over dispatches of the value summed over its hardware instances, instances per dispatch),
    for kernels whose name matches the regular expression kernel_substr."""
    con = sqlite3.connect(db)
    per = {c: {} for c in counters}
    inst = {c: {} for c in counters}
    for name, disp, cn, v in con.execute("select name, dispatch_id, counter_name, counter_value from pmc_events"):
        if cn in per and re.search(kernel_substr, name.replace(" ", "")):
            per[cn][disp] = per[cn].get(disp, 0.0) + v
            inst[cn][disp] = inst[cn].get(disp, 0) + 1
    out = {}
    for c in counters:
        if not per[c]:
            raise RuntimeError(f"no {c} samples for {kernel_substr} in {db}")
        out[c] = (float(np.mean(list(per[c].values()))), int(max(inst[c].values())))
    return out


def _profile_counters(counters: list[str], child_args: list[str], kernel_substr: str, timeout: int = 150) -> dict:
    with tempfile.TemporaryDirectory() as tmp:
        cmd = ["rocprofv3", "--pmc", *counters, "-d", tmp, "-o", "run", "--", sys.executable, str(HERE / "bench.py"),
               "--pmc-child", *child_args]
        subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=timeout, check=True)
        dbs = sorted(Path(tmp).rglob("*results.db"))
        if not dbs:
            raise RuntimeError("rocprofv3 wrote no results database")
        return _counters_per_dispatch(dbs[0], counters, kernel_substr)


def _profile(counter: str, child_args: list[str], kernel_substr: str, timeout: int = 150) -> float:
    return _profile_counters([counter], child_args, kernel_substr, timeout)[counter][0]


BUSY_COUNTERS = ["SQ_INSTS_MFMA", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY",
                 "GRBM_GUI_ACTIVE"]


def pmc_busy(config: str, simds: int) -> dict:
    """Issue counters of the experts launch, one rocprofv3 pass: MFMA pipe busy as a fraction of every SIMD's cycles
    over the dispatch (SQ_VALU_MFMA_BUSY_CYCLES sums the busy cycles of all SIMDs; GRBM_GUI_ACTIVE counts the
    dispatch's cycles once per instance), MFMA and VALU instructions (per wave64 instruction) and the share of wave
    cycles spent waiting for an instruction's operands or a barrier."""
    c = _profile_counters(BUSY_COUNTERS, ["--config", config], EXPERTS_KERNEL)
    cycles = c["GRBM_GUI_ACTIVE"][0] / c["GRBM_GUI_ACTIVE"][1]
    return {"mfma_insts": c["SQ_INSTS_MFMA"][0], "valu_insts": c["SQ_INSTS_VALU"][0], "cycles": cycles,
            "mfma_busy_frac": c["SQ_VALU_MFMA_BUSY_CYCLES"][0] / (simds * cycles),
            "wave_wait_frac": c["SQ_WAIT_INST_ANY"][0] / max(c["SQ_WAVE_CYCLES"][0], 1.0),
            "command": f"rocprofv3 --pmc {' '.join(BUSY_COUNTERS)} -d <dir> -o run -- python3 bench.py --pmc-child "
                       f"--config {config}"}


def pmc_traffic(config: str) -> dict:
    """HBM bytes per experts launch from FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled by the ratio of
    the known bytes of a COPY_MIB MiB device copy to what the same counter reads for it."""
    copy_bytes = COPY_MIB << 20
    fetch_copy = _profile("FETCH_SIZE", ["--copy-calibration", str(COPY_MIB)], "copyBuffer")
    write_copy = _profile("WRITE_SIZE", ["--copy-calibration", str(COPY_MIB)], "copyBuffer")
    f_fetch, f_write = copy_bytes / (fetch_copy * 1024), copy_bytes / (write_copy * 1024)
    fetch = _profile("FETCH_SIZE", ["--config", config], EXPERTS_KERNEL) * 1024 * f_fetch
    write = _profile("WRITE_SIZE", ["--config", config], EXPERTS_KERNEL) * 1024 * f_write
    return {"fetch_bytes": fetch, "write_bytes": write, "fetch_scale": f_fetch, "write_scale": f_write}


# ---- the measurement --------------------------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="headline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-pmc", action="store_true", help="skip the rocprofv3 traffic passes (traffic: null)")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--copy-calibration", type=int, default=0, help=argparse.SUPPRESS)
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this MoE layer runs on a single MI355X by design (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE {world}); run it with --gpus 1", file=sys.stderr)
        return 2
    if args.pmc_child:
        return _pmc_child(args)

    from janus_amd import _lib

    dev = torch.device("cuda", 0)
    cfg, layer, x, blk = make_layer(args.config, dev)
    with torch.no_grad():
        blk(x)                                  # router prep, first launch
        _, _, idx = blk.gate(x)
    torch.cuda.synchronize()
    idx_np = idx.cpu().numpy()
    work = layer_work(cfg, idx_np)
    rows = np.bincount(idx_np.reshape(-1), minlength=cfg.E)
    routing = {"experts_hit": int(np.count_nonzero(rows)), "max_rows": int(rows.max()),
               "mean_rows": float(rows.mean()), "max_over_mean": float(rows.max() / rows.mean())}
    L = _lib.lib()

    def step():
        with torch.no_grad():
            return blk(x)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K eager forwards back to back, bracketed by device synchronisation
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed / args.steps * 1e3

    # the stage breakdown, in K more forwards that each record their own stage events on the launch stream (each event
    # is a command-processor packet between two kernels, a few us per step in all, so these steps are kept out of
    # `value`)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(STAGES) + 1)] for _ in range(args.steps)]
    for row in events:
        for e in row:
            e.record()                          # creates the underlying hipEvent
    handles = [(ctypes.c_void_p * len(row))(*[ctypes.c_void_p(e.cuda_event) for e in row]) for row in events]
    torch.cuda.synchronize()
    for i in range(args.steps):
        L.janus_moe_profile_events(handles[i], len(STAGES) + 1)
        step()
    L.janus_moe_profile_events(None, 0)
    torch.cuda.synchronize()
    stage_ms = np.array([[row[j].elapsed_time(row[j + 1]) for j in range(len(STAGES))] for row in events])
    raw_us = {n: float(v) * 1e3 for n, v in zip(STAGES, stage_ms.mean(0))}
    split = os.environ.get("JANUS_MOE_SCHEDULE") == "split"
    stage_us = {"route": raw_us["route"], "align": raw_us["align"], "experts": raw_us["gate_up"] + raw_us["down"],
                "combine": raw_us["combine"]}
    if split:
        stage_us.update(gate_up=raw_us["gate_up"], down=raw_us["down"])

    # the same forward replayed from a HIP graph (the reference serves under graphs)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_s = (time.perf_counter() - t1) / args.steps

    ex_s = stage_us["experts"] * 1e-6
    t_step = ms * 1e-3
    t_roof = max(work["flops"] / MFMA_BF16_PEAK, work["bytes"] / HBM_PEAK)
    if work["ex_bytes"] / HBM_PEAK >= work["ex_flops"] / MFMA_BF16_PEAK:
        ach = work["ex_bytes"] / ex_s / 1e9
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": ach / (HBM_PEAK / 1e9)}
    else:
        ach = work["ex_flops"] / ex_s / 1e12
        roof = {"bound": "mfma", "achieved": ach, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": ach / (MFMA_BF16_PEAK / 1e12)}
    traffic, traffic_note = None, "skipped (--no-pmc)"
    if split:
        traffic_note = "skipped: JANUS_MOE_SCHEDULE=split runs the GEMMs as two launches"
    elif not args.no_pmc:
        try:
            t = pmc_traffic(args.config)
            traffic = t["fetch_bytes"] + t["write_bytes"]
            traffic_note = (f"rocprofv3 FETCH_SIZE x {t['fetch_scale']:.3f} + WRITE_SIZE x {t['write_scale']:.3f} "
                            f"(scales from a {COPY_MIB} MiB copy): fetch {t['fetch_bytes']:.4g} B, "
                            f"write {t['write_bytes']:.4g} B per launch")
        except Exception as exc:  # no profiler on this machine: the entry stays null, with the reason
            traffic_note = f"unavailable: {type(exc).__name__}: {exc}"[:300]
    busy = None
    if not split and not args.no_pmc:
        try:
            busy = pmc_busy(args.config, 4 * torch.cuda.get_device_properties(dev).multi_processor_count)
        except Exception as exc:
            busy = f"unavailable: {type(exc).__name__}: {exc}"[:300]
    kernel = "w4a16_gemm_kernel<gate_up> + <down> (split)" if split else "moe_experts_kernel (gate_up + down)"
    roof.update({"traffic": traffic, "kernel": kernel, "algorithmic_bytes": work["ex_bytes"],
                 "algorithmic_flops": work["ex_flops"], "avg_us": stage_us["experts"], "traffic_source": traffic_note,
                 "issue_counters": busy})

    result = {
        "metric": METRIC, "value": cfg.T / t_step, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: seeded splitmix64 activations and random int4 g128 weights",
        "config": {"workload": f"W4A16 MoE layer {cfg.name}: T={cfg.T} H={cfg.H} E={cfg.E} top{cfg.k} I={cfg.I} "
                               f"shared I={cfg.I_s}", "T": cfg.T, "H": cfg.H, "experts": cfg.E, "top_k": cfg.k,
                   "I": cfg.I, "I_shared": cfg.I_s, "codec": "int4 group-128, bf16 scales",
                   "timing": "eager launches on one stream, stage events per step"},
        "roofline": roof,
        "layer_roofline": {"t_roof_us": t_roof * 1e6, "t_us": t_step * 1e6, "frac": t_roof / t_step,
                           "bound": "hbm" if work["bytes"] / HBM_PEAK >= work["flops"] / MFMA_BF16_PEAK else "mfma",
                           "flops": work["flops"], "bytes": work["bytes"], "n_hit": work["n_hit"]},
        "stages_us": stage_us,
        "routing": routing,
        "graph_tokens_per_s": cfg.T / graph_s, "graph_ms_per_step": graph_s * 1e3,
    }
    result["variants_us"] = variant_timings(cfg, x, blk, dev)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(layer, x, cfg.k, step())
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
