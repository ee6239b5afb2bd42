"""Benchmark of the HIP Pairformer path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config C2] [--no-cpu-baseline]

A step is one forward pass of the configured workload over synthetic inputs already in
HBM: C2 (default, the metric's N=384 configuration) = one Pairformer pair block at N=384
in bf16; C1 = the same at N=128 in fp32; C3 = the 48-block trunk at N=768 (single track
included); C4 = the 24-block diffusion transformer, 5 samples, N=768; C5 = one pair block
at N=1536. ``value`` is milliseconds per Pairformer block (per transformer pass for C4).

Rank 0 prints one JSON line with the driver's fields plus ``roofline`` (the dominant
kernel, timed with HIP events on its own stream inside this run) and ``cpu_baseline``
(the CPU oracle, a restatement of the reference's torch backend, on a bounded sample).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ms per Pairformer block at N=384/768 bf16; MFMA util % and HBM GB/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


# (timed steps, warm-up steps) per configuration; a step is one forward of the workload.
DEFAULT_STEPS = {"C1": (200, 50), "C2": (200, 50), "C3": (10, 3), "C4": (10, 3), "C5": (20, 5)}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default per config: enough to reach steady clocks)")
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--graph", action="store_true",
                   help="capture one step in a HIP graph after the warm-up and time its replays")
    p.add_argument("--copy-calibration-mb", type=int, default=0,
                   help="after the run, read and write a buffer of this many MiB once (a plain copy "
                        "kernel of known size whose FETCH_SIZE/WRITE_SIZE counters calibrate the "
                        "traffic figure)")
    args = p.parse_args()
    # A single N=384 block is ~0.7 ms: a few warm-up blocks leave the GPU below its steady
    # clock, so the small configurations warm up and time over many blocks.
    steps, warmup = DEFAULT_STEPS[args.config]
    args.steps = steps if args.steps is None else args.steps
    args.warmup = warmup if args.warmup is None else args.warmup
    return args


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def build_workload(cfg_name, device):
    import torch
    from xfold_cpu_amd import nn as hnn
    from xfold_cpu_amd.synthetic import CONFIGS, diffusion_inputs, init_module_, pair_block_inputs

    cfg = CONFIGS[cfg_name]
    bf16 = cfg["dtype"] == "bf16"
    if cfg["kind"] in ("pair_block", "trunk"):
        blocks = cfg.get("blocks", 1)
        with_single = cfg["with_single"]
        mods = []
        for b in range(blocks):
            m = hnn.PairformerBlock(n_heads=16, c_pair=128, c_single=384, n_heads_pair=4,
                                    with_single=with_single).eval()
            init_module_(m, seed=b)
            mods.append(m.to(device))
        inp = pair_block_inputs(cfg["n"], pad=cfg["pad"], random_pad=cfg["random_pad"], seed=0,
                                with_single=with_single)
        dt = torch.bfloat16 if bf16 else torch.float32
        pair0 = inp.pair.to(dt).to(device)
        single0 = inp.single.to(dt).to(device) if with_single else None
        pmask, smask = inp.pair_mask.to(device), inp.seq_mask.to(device)
        state = {"pair": pair0.clone(), "single": single0.clone() if with_single else None}

        def step():
            with torch.inference_mode(), torch.amp.autocast("cuda", dtype=torch.bfloat16, enabled=bf16):
                for m in mods:
                    if with_single:
                        m(state["pair"], pmask, state["single"], smask)
                    else:
                        m(state["pair"], pmask)

        workload = dict(workload=f"{cfg_name}: {blocks} Pairformer block(s), N={cfg['n']}, "
                                 f"{'single track, ' if with_single else 'pair stack, '}"
                                 f"{cfg['pad']} padded tokens", n_tokens=cfg["n"], blocks=blocks,
                        c_pair=128, heads_pair="4x32", pair_transition="128->2x512->128")
        return step, blocks, workload, cfg
    # diffusion transformer
    m = hnn.DiffusionTransformer().eval()
    init_module_(m, seed=0)
    m.to(device)
    inp = diffusion_inputs(cfg["n"], samples=cfg["samples"])
    act0 = inp.act.bfloat16().to(device)
    mask, scond, pcond = inp.mask.to(device), inp.single_cond.to(device), inp.pair_cond.to(device)
    state = {"act": act0.clone()}

    def step():
        with torch.inference_mode(), torch.amp.autocast("cuda", dtype=torch.bfloat16):
            m(state["act"], mask, scond, pcond)

    workload = dict(workload=f"C4: diffusion transformer, 24 blocks, {cfg['samples']} samples, N={cfg['n']}",
                    n_tokens=cfg["n"], blocks=24, samples=cfg["samples"])
    return step, 1, workload, cfg


# HBM bytes per grid_attention_kernel launch, from rocprofv3 FETCH_SIZE and WRITE_SIZE passes over
# the same workload (bench.py --config C2|C3 --copy-calibration-mb 512), calibrated against that
# 512 MiB read+write kernel: bytes = (2 x FETCH_SIZE + WRITE_SIZE) KiB x 1024. Counters cannot be
# read inside this process, so the figure is the recorded measurement for the configuration.
ATTENTION_TRAFFIC_BYTES = {384: 168.25e6, 768: 1037.9e6}


PAIR_TIMERS = ("transition", "trimul_project", "trimul_contract", "trimul_output", "grid_project",
               "grid_attention", "grid_output", "pair_bias")


def kernel_roofline(step, n, steps):
    """Average launch duration of every pair-stack kernel inside the block workload, from HIP
    events the library records around each launch on the launch stream, with its HBM or MFMA
    rate (algorithmic bytes / FLOPs of one launch, xfold_cpu_amd.kernel_bench). Returns the
    roofline object of the dominant kernel (triangle attention core: B=N rows, 4 heads x 32,
    N x N keys, pair bias and 2-D key mask) and the per-kernel table."""
    import torch
    from xfold_cpu_amd.fastnn import native_hip
    from xfold_cpu_amd.kernel_bench import pair_kernel_work, rates

    for name in PAIR_TIMERS:
        native_hip.kernel_timing_read(name)           # drop anything recorded earlier
    native_hip.set_kernel_timing(True)
    try:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        native_hip.set_kernel_timing(False)
    timed = {name: native_hip.kernel_timing_read(name) for name in PAIR_TIMERS}
    work = pair_kernel_work(n)
    kernels = {}
    for name, (total_ms, launches) in timed.items():
        if launches:
            kernel, gbytes, gflop = work[name]
            r = rates(total_ms / launches, gbytes, gflop)
            kernels[kernel] = dict(avg_us=round(total_ms / launches * 1e3, 2), launches=launches,
                                   **{k: r[k] for k in ("hbm_tbs", "hbm_frac", "tflops", "mfma_frac") if k in r})
    total_ms, launches = timed["grid_attention"]
    if launches == 0:
        return None, kernels
    ms = total_ms / launches
    heads, d = 4, 32
    flops = 4.0 * n * heads * n * n * d            # Q.K^T and P.V over all N^3 logits
    achieved = flops / (ms * 1e-3) / 1e12
    return {"kernel": "grid_attention_kernel (triangle attention core)", "bound": "mfma",
            "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": ATTENTION_TRAFFIC_BYTES.get(n),
            "avg_launch_ms": round(ms, 4), "launches": launches, "flops_per_launch": flops,
            "shape": f"B={n} H={heads} Q=K={n} D={d} bf16"}, kernels


def cpu_baseline(cfg, budget_s=30.0):
    """The CPU oracle (restatement of the reference's torch backend) on the host cores:
    one Pairformer pair block at the configuration's N under CPU bf16 autocast (fp32 for
    C1), or the largest N in {N, 256, 128} whose single run fits the time budget."""
    import torch
    from oracle import restatement as R
    from xfold_cpu_amd.synthetic import init_module_, pair_block_inputs

    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cores = min(cores, 16)
    torch.set_num_threads(cores)
    bf16 = cfg["dtype"] == "bf16"
    n_full = cfg["n"] if cfg["kind"] != "diffusion" else 384
    for n in (n_full, 256, 128):
        if n > 384:
            continue
        block = init_module_(R.PairformerBlock(with_single=False).eval(), seed=0)
        inp = pair_block_inputs(n, pad=max(1, n // 12), seed=0, with_single=False)
        pair = inp.pair.bfloat16() if bf16 else inp.pair
        attention = R.dot_product_attention_chunked
        t0 = time.perf_counter()
        with torch.inference_mode(), torch.amp.autocast("cpu", dtype=torch.bfloat16, enabled=bf16):
            block(pair.clone(), inp.pair_mask, attention=lambda *a, **k: attention(*a, rows_per_chunk=32, **k))
        dt = time.perf_counter() - t0
        if dt <= budget_s or n == 128:
            return {"value": round(dt * 1e3, 1), "unit": "ms per Pairformer pair block", "cores": cores,
                    "kind": "port",
                    "sample": f"1 pair block (TriMul out/in, TriAtt start/end, Transition) at N={n}, "
                              f"{'bf16 CPU autocast' if bf16 else 'fp32'}, torch CPU restatement "
                              f"of the reference torch backend, {cores} threads"}
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU figures are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from xfold_cpu_amd.fastnn import native_hip

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm device")
    native_hip.load_library()
    device = torch.device("cuda:0")
    log(f"config {args.config}: building workload")
    step, blocks, workload, cfg = build_workload(args.config, device)
    for i in range(args.warmup):
        step()
        if i == 0 or i + 1 == args.warmup:
            log(f"warmup {i + 1}/{args.warmup}")
    torch.cuda.synchronize()
    run = step
    if args.graph:
        # The step records no memset, host copy or synchronisation, so it replays as a graph.
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        run = graph.replay
        log("captured one step in a HIP graph")
    stream = torch.cuda.current_stream(device)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        run()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(stop) / args.steps
    log(f"timed {args.steps} steps: {ms_step:.3f} ms/step (wall {wall:.2f} s)")
    value = ms_step / blocks

    roof, kernels = None, None
    if cfg["kind"] != "diffusion":
        roof, kernels = kernel_roofline(step, cfg["n"], max(1, min(args.steps, 5)))
        log(f"roofline: {roof}")
    base = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)")
        base = cpu_baseline(cfg)
        log(f"cpu baseline: {base}")

    if args.copy_calibration_mb:
        # One elementwise kernel (bitwise_not, a name no other kernel of the run has) that
        # reads and writes exactly this many MiB.
        src = torch.ones(args.copy_calibration_mb << 20, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        log(f"copy calibration: {args.copy_calibration_mb} MiB read and written")

    dtype = "bf16" if cfg["dtype"] == "bf16" else "fp32"
    line = {
        "metric": METRIC, "value": round(value, 4), "unit": "ms", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded N(0,1) activations, N(0,1/fan_in) weights)",
        "config": dict(workload, launch="hip graph replay" if args.graph else "eager"),
        "roofline": roof, "cpu_baseline": base, "kernels": kernels,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
