"""Benchmark of the HIP Pairformer path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config C2] [--no-cpu-baseline]
                    [--no-c3] [--no-c4] [--no-c5] [--no-cached] [--graph]

A step is one forward pass of the configured workload over synthetic inputs already in
HBM: C2 (default, the metric's N=384 configuration) = one Pairformer pair block at N=384
in bf16; C1 = the same at N=128 in fp32; C3 = the 48-block trunk at N=768 (single track
included); C4 = the 24-block diffusion transformer, 5 samples, N=768; C5 = one pair block
at N=1536. ``value`` is milliseconds per Pairformer block (per transformer pass for C4).

One JSON line with the driver's fields plus ``roofline`` (the dominant kernel, timed with
HIP events on its launch stream inside this run; ``traffic`` from the rocprofv3 counter
record of the same kernel sources), ``kernels`` (every pair kernel's rate) and
``cpu_baseline`` (restatements of the reference's torch and cpp backends timed on the host
cores: 1 warm-up, median of 3). With the default C2 configuration the other GPU
configurations are timed in the same run, each with its own roofline, kernels and CPU
legs: ``c3`` (the 48-block N=768 trunk, the north-star target), ``c4`` (the diffusion
transformer, uncached and inside an input-cache scope) and ``c5`` (the N=1536 block).
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
DEFAULT_STEPS = {"C1": (200, 50), "C2": (200, 50), "C3": (5, 2), "C4": (10, 3), "C5": (20, 5), "T768": (20, 5)}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default per config: enough to reach steady clocks)")
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5", "T768"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-c3", action="store_true",
                   help="with the default C2 configuration, skip the 48-block C3 trunk timed beside it")
    p.add_argument("--no-c4", action="store_true",
                   help="with the default C2 configuration, skip the C4 diffusion transformer timed beside it")
    p.add_argument("--no-c5", action="store_true",
                   help="with the default C2 configuration, skip the C5 N=1536 block timed beside it")
    p.add_argument("--no-cached", action="store_true",
                   help="with C4, skip the input-cache forward timed beside the uncached one")
    p.add_argument("--precondition-s", type=float, default=0.3,
                   help="after each configuration's first warm-up step (which builds the weight "
                        "caches while the GPU idles), run this many seconds of large bf16 GEMMs "
                        "(torch.matmul, not the workload) so that the GPU leaves its idle clock "
                        "state; 0 disables it")
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
        c_pair, factor = cfg.get("c_pair", 128), cfg.get("factor", 4)
        mods = []
        for b in range(blocks):
            m = hnn.PairformerBlock(n_heads=16, c_pair=c_pair, c_single=384, n_heads_pair=4,
                                    with_single=with_single, num_intermediate_factor=factor).eval()
            init_module_(m, seed=b)
            mods.append(m.to(device))
        inp = pair_block_inputs(cfg["n"], c_pair=c_pair, pad=cfg["pad"], random_pad=cfg["random_pad"], seed=0,
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
                        c_pair=c_pair, heads_pair=f"4x{c_pair // 4}",
                        pair_transition=f"{c_pair}->2x{factor * c_pair}->{c_pair}")
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
                    n_tokens=cfg["n"], blocks=24, samples=cfg["samples"],
                    input_cache="off in the timed steps (pair logits and conditioning recomputed per forward)")
    return step, 1, workload, cfg


def time_cached_diffusion(step, steps, warmup):
    """ms per C4 forward inside an input-cache scope (the reference's InputCache rules, as
    its sampler runs 200 forwards per example): the packed pair logits of all 24 blocks are
    computed in the first forward and reused. Reported beside the uncached time."""
    import torch
    from xfold_cpu_amd.fastnn import config
    from xfold_cpu_amd.nn.cache import input_cache_scope
    saved = config.input_cache_enabled
    config.input_cache_enabled = True
    try:
        with torch.no_grad(), input_cache_scope():
            for _ in range(warmup):
                step()
            torch.cuda.synchronize()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(steps):
                step()
            stop.record()
            torch.cuda.synchronize()
    finally:
        config.input_cache_enabled = saved
    return start.elapsed_time(stop) / steps


COUNTER_FILES = {"C2": ROOT / "profiles" / "counters_c2_n384.md", "C3": ROOT / "profiles" / "counters_c3_n768.md",
                 "C4": ROOT / "profiles" / "counters_c4_n768.md", "C5": ROOT / "profiles" / "counters_c5_n1536.md"}


def recorded_traffic(cfg_name, kernel):
    """HBM bytes per launch of ``kernel`` in configuration ``cfg_name``, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE passes recorded in profiles/counters_*.md (calibrated against a
    512 MiB read+write kernel in the same run). Counters cannot be read inside this process,
    so the figure is the recorded measurement; it is returned only while the kernel's
    sources hash to the digest recorded with it, else (None, reason)."""
    import hashlib
    path = COUNTER_FILES.get(cfg_name)
    if path is None or not path.exists():
        return None, f"no counter record for {cfg_name}"
    rec = None
    for line in path.read_text().splitlines():
        if line.startswith(f'{{"counters": "{kernel}"'):
            rec = json.loads(line)
    if rec is None:
        return None, f"{path.name} holds no machine-readable record for {kernel}"
    h = hashlib.sha256()
    for src in rec["sources"]:
        h.update((ROOT / src).read_bytes())
    if h.hexdigest() != rec["sources_sha256"]:
        return None, (f"stale: {path.name} was measured at commit {rec['commit']} on other {kernel} "
                      "sources")
    return rec["traffic_bytes"], f"{path.name} (commit {rec['commit']}, sources match)"


PAIR_TIMERS = ("transition", "trimul_project", "trimul_contract", "trimul_output", "grid_project",
               "grid_attention", "grid_output", "pair_bias")


def kernel_roofline(step, cfg_name, n, steps):
    """Average launch duration of every pair-stack kernel inside the block workload, from HIP
    events the library records around each launch on the launch stream, with its HBM or MFMA
    rate (algorithmic bytes / FLOPs of one launch, xfold_cpu_amd.kernel_bench). Returns the
    roofline object of the dominant kernel (triangle attention core: B=N rows, 4 heads x 32,
    N x N keys, pair bias and 2-D key mask) and the per-kernel table."""
    import torch
    from xfold_cpu_amd.fastnn import native_hip
    from xfold_cpu_amd.kernel_bench import pair_kernel_work, rates

    native_hip.set_kernel_timing(True)
    try:
        # One step with the timers on is dropped: the first event records of a process
        # read up to 15% high on a fresh box. The timed steps follow at once: the timers
        # are the dispatches' own start and end, so host submission does not enter them,
        # and an idle wait before the steps (a spin kernel was used here) lets the clocks
        # drop: measured on C2, the kernels then summed to 582-598 us per 545 us block,
        # without it to 536 us per 547 us block.
        step()
        torch.cuda.synchronize()
        for name in PAIR_TIMERS:
            native_hip.kernel_timing_read(name)       # drop it and anything recorded earlier
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
    traffic, traffic_src = recorded_traffic(cfg_name, "grid_attention_kernel")
    return {"kernel": "grid_attention_kernel (triangle attention core)", "bound": "mfma",
            "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic, "traffic_source": traffic_src,
            "avg_launch_ms": round(ms, 4), "launches": launches, "flops_per_launch": flops,
            "shape": f"B={n} H={heads} Q=K={n} D={d} bf16"}, kernels


DIFFUSION_TIMERS = ("gemm_ring", "mha_attention", "pair_bias", "layer_norm")


def diffusion_roofline(step, cfg_name, steps):
    """The diffusion transformer's kernels inside its forward: average launch time and the
    rate of the algorithmic FLOPs each launch declares (every Linear's 2 M N K for gemm_ring,
    4 B H N^2 Dv for the attention), from HIP events on the launch stream. The roofline
    object is the dominant kernel, gemm_ring (all Linears of the forward aggregated: their
    FLOPs over their summed launch time)."""
    import torch
    from xfold_cpu_amd.fastnn import native_hip

    native_hip.set_kernel_timing(True)
    try:
        step()                                        # dropped: a process's first event records read high
        torch.cuda.synchronize()
        for name in DIFFUSION_TIMERS:
            native_hip.kernel_timing_read_work(name)
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        native_hip.set_kernel_timing(False)
    kernels = {}
    for name in DIFFUSION_TIMERS:
        total_ms, launches, work = native_hip.kernel_timing_read_work(name)
        if not launches:
            continue
        rec = dict(avg_us=round(total_ms / launches * 1e3, 2), launches=launches,
                   ms_per_forward=round(total_ms / steps, 4))
        if work:
            tflops = work / (total_ms * 1e-3) / 1e12
            rec.update(tflops=round(tflops, 1), mfma_frac=round(tflops / PEAK_BF16_TFLOPS, 4))
        kernels[name + "_kernel"] = rec
    g = kernels.get("gemm_ring_kernel")
    if g is None:
        return None, kernels
    ms_all = g["ms_per_forward"] * steps
    flops = g["tflops"] * 1e12 * ms_all * 1e-3
    traffic, traffic_src = recorded_traffic(cfg_name, "gemm_ring_kernel")
    return {"kernel": "gemm_ring_kernel (every Linear of the forward, aggregated over its shapes)",
            "bound": "mfma", "achieved": g["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(g["tflops"] / PEAK_BF16_TFLOPS, 4), "traffic": traffic, "traffic_source": traffic_src,
            "avg_launch_ms": round(g["avg_us"] / 1e3, 4), "launches": g["launches"],
            "flops_per_launch": round(flops / g["launches"]),
            "shape": "per block: [5*768, 768] x 768->3072 (q, k, v, gate), 768->768 (AdaLNZero), "
                     "768->3072 (GLU), 1536->768; plus the batched conditioning Linears"}, kernels


WIDTH_TIMERS = ("mha_attention", "gemm_ring", "layer_norm")


def width_roofline(step, n, steps):
    """A pair block off the 128-channel fast path (the template stack's): the timed kernels'
    average launch time per block and their declared FLOP rates; the roofline object is the
    attention (the pipelined kernel on repacked operands, 4 B H N^2 Dv FLOPs per launch)."""
    import torch
    from xfold_cpu_amd.fastnn import native_hip

    native_hip.set_kernel_timing(True)
    try:
        step()                                        # dropped: a process's first event records read high
        torch.cuda.synchronize()
        for name in WIDTH_TIMERS:
            native_hip.kernel_timing_read_work(name)
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        native_hip.set_kernel_timing(False)
    kernels = {}
    for name in WIDTH_TIMERS:
        total_ms, launches, work = native_hip.kernel_timing_read_work(name)
        if not launches:
            continue
        rec = dict(avg_us=round(total_ms / launches * 1e3, 2), launches=launches,
                   us_per_block=round(total_ms / steps * 1e3, 1))
        if work:
            tflops = work / (total_ms * 1e-3) / 1e12
            rec.update(tflops=round(tflops, 1), mfma_frac=round(tflops / PEAK_BF16_TFLOPS, 4))
        kernels[name + "_kernel"] = rec
    a = kernels.get("mha_attention_kernel")
    if a is None or "tflops" not in a:
        return None, kernels
    return {"kernel": "grid_attention_kernel on repacked operands (mha_attention)", "bound": "mfma",
            "achieved": a["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": a["mfma_frac"], "traffic": None, "traffic_source": "no counter record for this configuration",
            "avg_launch_ms": round(a["avg_us"] / 1e3, 4), "launches": a["launches"],
            "shape": f"B={n} H=4 Q=K={n} D=16 (padded to 32) bf16"}, kernels


def host_cpu():
    """CPU model, sockets, cores and SMT of the host (lscpu), and the cores this process may use."""
    import subprocess
    info = {"affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        out = ""
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "CPU(s)": "cpus"}
    for line in out.splitlines():
        key, _, value = line.partition(":")
        if key.strip() in keys:
            value = value.strip()
            info[keys[key.strip()]] = int(value) if value.isdigit() else value
    return info


def cpu_threads():
    """Threads for the CPU legs: every core of this process's affinity, capped at the host share
    the job was given (OMP_NUM_THREADS, set to one GPU's share of the box's cores)."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    share = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(affinity, int(share))) if share.isdigit() else affinity


def _median_ms(fn, runs=3, warmup=1):
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    return times[len(times) // 2], [round(t, 1) for t in times]


def cpu_workload(cfg_name, leg):
    """(callable, description, blocks per call, extrapolation factor) of the CPU restatement of
    one configuration. ``leg`` "torch": oracle.restatement (the reference's torch backend);
    "cpp": oracle.cpp_port (the af3_kernels algorithms, OpenMP tiles over ATen GEMMs)."""
    import torch
    from oracle import restatement as R
    from xfold_cpu_amd.synthetic import CONFIGS, diffusion_inputs, init_module_, pair_block_inputs

    cfg = CONFIGS[cfg_name]
    bf16 = cfg["dtype"] == "bf16"
    autocast = lambda: torch.amp.autocast("cpu", dtype=torch.bfloat16, enabled=bf16)  # noqa: E731
    if leg == "cpp":
        from oracle import cpp_port
        cpp_port.load()
    if cfg["kind"] == "diffusion":
        m = init_module_(R.DiffusionTransformer().eval(), seed=0)
        inp = diffusion_inputs(cfg["n"], samples=cfg["samples"])
        act = inp.act.bfloat16().float() if bf16 else inp.act
        run_module = m if leg == "torch" else cpp_port.DiffusionTransformerCpp(m)

        def fn():
            with torch.inference_mode(), autocast():
                for s in range(cfg["samples"]):
                    run_module(act[s].clone(), inp.mask, inp.single_cond, inp.pair_cond)
        return fn, f"24-block diffusion transformer, {cfg['samples']} samples, N={cfg['n']}", 1, 1
    with_single = cfg["with_single"]
    block = init_module_(R.PairformerBlock(with_single=with_single).eval(), seed=0)
    inp = pair_block_inputs(cfg["n"], pad=cfg["pad"], random_pad=cfg["random_pad"], seed=0, with_single=with_single)
    pair = inp.pair.bfloat16() if bf16 else inp.pair
    single = (inp.single.bfloat16() if bf16 else inp.single) if with_single else None
    chunked = lambda *a, **k: R.dot_product_attention_chunked(*a, rows_per_chunk=32, **k)  # noqa: E731
    run_block = block if leg == "torch" else cpp_port.PairformerBlockCpp(block)

    def fn():
        with torch.inference_mode(), autocast():
            if with_single:
                run_block(pair.clone(), inp.pair_mask, single.clone(), inp.seq_mask, attention=chunked)
            else:
                run_block(pair.clone(), inp.pair_mask, attention=chunked)
    blocks = cfg.get("blocks", 1)
    what = (f"one Pairformer block at N={cfg['n']}{' with single track' if with_single else ' (pair stack)'}, "
            f"{'bf16 CPU autocast' if bf16 else 'fp32'}")
    return fn, what, 1, blocks


C5_SAMPLE_ROWS = (32, 96)


def cpu_c5_sample(leg):
    """C5 (one pair block at N=1536) on the host, bounded: both triangle multiplications and
    the transition in full; each triangle-attention node on 32 and on 96 of its 1536 batch
    rows, extrapolated linearly to all rows (every batch row costs the same: its own N x N
    logits per head over the shared bias; the intercept is the full LayerNorm and bias
    projection). One timed run of each part after a warm-up pair block at N=64. Returns
    (ms per block, parts, description)."""
    import torch
    from oracle import restatement as R
    from xfold_cpu_amd.synthetic import CONFIGS, init_module_, pair_block_inputs

    cfg = CONFIGS["C5"]
    n = cfg["n"]
    block = init_module_(R.PairformerBlock(with_single=False).eval(), seed=0)
    if leg == "cpp":
        from oracle import cpp_port
        cpp_port.load()
        tri = cpp_port.triangle_multiplication_cpp
        rows_fn = cpp_port.grid_self_attention_rows_cpp
        trans = cpp_port.transition_cpp
        warm = cpp_port.PairformerBlockCpp(block)
    else:
        tri = lambda m, p, mask: m(p, mask)  # noqa: E731
        rows_fn = R.grid_self_attention_rows
        trans = lambda m, p: m(p)  # noqa: E731
        warm = block
    autocast = lambda: torch.amp.autocast("cpu", dtype=torch.bfloat16)  # noqa: E731
    small = pair_block_inputs(64, pad=4, seed=0, with_single=False)
    chunked = lambda *a, **k: R.dot_product_attention_chunked(*a, rows_per_chunk=32, **k)  # noqa: E731
    with torch.inference_mode(), autocast():
        warm(small.pair.bfloat16(), small.pair_mask, attention=chunked)
    inp = pair_block_inputs(n, pad=cfg["pad"], random_pad=cfg["random_pad"], seed=0, with_single=False)
    pair, mask = inp.pair.bfloat16(), inp.pair_mask

    def timed(fn):
        t0 = time.perf_counter()
        with torch.inference_mode(), autocast():
            fn()
        return (time.perf_counter() - t0) * 1e3
    parts = {}
    parts["triangle_multiplication_outgoing"] = timed(lambda: tri(block.triangle_multiplication_outgoing, pair, mask))
    parts["triangle_multiplication_incoming"] = timed(lambda: tri(block.triangle_multiplication_incoming, pair, mask))
    for node in ("pair_attention1", "pair_attention2"):
        module = getattr(block, node)
        (r0, r1) = C5_SAMPLE_ROWS
        t0 = timed(lambda: rows_fn(module, pair, mask, torch.arange(r0)))
        t1 = timed(lambda: rows_fn(module, pair, mask, torch.arange(r0, r0 + r1)))
        per_row = max(t1 - t0, 0.0) / (r1 - r0)
        parts[node] = t0 + per_row * (n - r0)
        parts[node + "_sample_ms"] = [round(t0, 1), round(t1, 1)]
    parts["pair_transition"] = timed(lambda: trans(block.pair_transition, pair))
    total = sum(v for k, v in parts.items() if not k.endswith("_sample_ms"))
    what = (f"one pair block at N={n}, bf16 CPU autocast: triangle multiplications and transition in full, "
            f"each attention node timed on {C5_SAMPLE_ROWS[0]} and {C5_SAMPLE_ROWS[1]} batch rows and "
            f"extrapolated linearly to {n}; one run per part after an N=64 warm-up block")
    return total, {k: (round(v, 1) if isinstance(v, float) else v) for k, v in parts.items()}, what


def cpu_baseline(cfg_name, runs=3):
    """The reference's CPU backends restated and timed on this host: 1 warm-up then the
    median of ``runs`` runs, on ``cpu_threads()`` threads (all cores of the affinity). The torch leg is
    oracle.restatement (the reference's torch backend); the cpp leg is oracle.cpp_port (the
    af3_kernels algorithms). ``value`` is the torch leg, in ms per Pairformer block (per
    transformer forward for C4); C3's 48-block figure is one block's time x 48."""
    import torch
    threads = cpu_threads()
    torch.set_num_threads(threads)
    legs = {}
    for leg in ("torch", "cpp"):
        if cfg_name == "C5":
            try:
                total, parts, what = cpu_c5_sample(leg)
            except (ImportError, RuntimeError, OSError) as err:
                legs[leg] = {"status": f"unavailable: {err}"}
                continue
            legs[leg] = {"ms_per_block": round(total, 1), "parts_ms": parts, "sample": what}
            log(f"cpu {leg}: {legs[leg]}")
            continue
        try:
            fn, what, per_call, factor = cpu_workload(cfg_name, leg)
        except (ImportError, RuntimeError, OSError) as err:
            legs[leg] = {"status": f"unavailable: {err}"}
            continue
        median, times = _median_ms(fn, runs=runs)
        rec = {"ms_per_block" if cfg_name != "C4" else "ms_per_forward": round(median / per_call, 1),
               "runs_ms": times, "sample": what}
        if factor > 1:
            rec["ms_per_trunk_extrapolated"] = round(median / per_call * factor, 1)
            rec["extrapolation"] = f"one block x {factor}"
        legs[leg] = rec
        log(f"cpu {leg}: {rec}")
    torch_leg = legs.get("torch", {})
    value = torch_leg.get("ms_per_block", torch_leg.get("ms_per_forward"))
    return {"value": value, "unit": "ms per Pairformer block" if cfg_name != "C4" else "ms per transformer forward",
            "cores": threads, "kind": "port",
            "sample": (f"{torch_leg.get('sample', cfg_name)}" +
                       ("" if cfg_name == "C5" else f"; 1 warm-up + median of {runs}") +
                       "; restatements of the reference's torch and cpp (af3_kernels) backends"),
            "legs": legs, "host": host_cpu()}


def precondition_clocks(device, seconds):
    """Runs ``seconds`` of 8192^3 bf16 GEMMs (torch.matmul; no part of the workload, nothing
    timed) so that the GPU leaves the low clock state it drops to while idle. The first
    warm-up step builds the weight caches on the host while the GPU idles; run after it,
    this brought 20 timed C2 blocks (5 warm-up blocks) from 0.612 to 0.554 ms per block on
    one box, where 200 blocks after 50 warm-up blocks take 0.552 ms. Run before the warm-up
    it changed nothing (the clocks drop again during the first step), and 1 s or 2 s of
    GEMMs gave no more than 0.3 s."""
    import torch
    if seconds <= 0:
        return
    a = torch.randn(8192, 8192, device=device, dtype=torch.bfloat16)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(4):
            torch.matmul(a, a)
        torch.cuda.synchronize()
    del a


def run_config(cfg_name, steps, warmup, device, graph=False, precondition_s=0.0):
    """Times ``steps`` steps of one configuration after ``warmup`` untimed ones (bracketed by
    device synchronisation, HIP events on the launch stream), then the per-kernel rooflines
    over a few more steps with the library's launch timers on. The GPU clocks are
    preconditioned (:func:`precondition_clocks`) after the first warm-up step."""
    import torch
    log(f"config {cfg_name}: building workload")
    step, blocks, workload, cfg = build_workload(cfg_name, device)
    if warmup == 0:
        precondition_clocks(device, precondition_s)
    for i in range(warmup):
        step()
        if i == 0:
            torch.cuda.synchronize()
            precondition_clocks(device, precondition_s)
        if i == 0 or i + 1 == warmup:
            log(f"{cfg_name} warmup {i + 1}/{warmup}")
    torch.cuda.synchronize()
    run = step
    if graph:
        # The step records no memset, host copy or synchronisation, so it replays as a graph.
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
        run = g.replay
        log("captured one step in a HIP graph")
    stream = torch.cuda.current_stream(device)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        run()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(stop) / steps
    log(f"{cfg_name} timed {steps} steps: {ms_step:.3f} ms/step (wall {wall:.2f} s)")
    roof, kernels = None, None
    if cfg.get("c_pair", 128) != 128:
        roof, kernels = width_roofline(step, cfg["n"], max(1, min(steps, 10)))
        log(f"{cfg_name} roofline: {roof}")
    elif cfg["kind"] != "diffusion":
        roof, kernels = kernel_roofline(step, cfg_name, cfg["n"], max(1, min(steps, 10)))
        log(f"{cfg_name} roofline: {roof}")
    else:
        roof, kernels = diffusion_roofline(step, cfg_name, max(1, min(steps, 10)))
        log(f"{cfg_name} roofline: {roof}")
    return dict(ms_step=ms_step, blocks=blocks, workload=workload, cfg=cfg, roofline=roof, kernels=kernels,
                step=step)


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
    res = run_config(args.config, args.steps, args.warmup, device, graph=args.graph,
                     precondition_s=args.precondition_s)
    ms_step, blocks, cfg = res["ms_step"], res["blocks"], res["cfg"]
    value = ms_step / blocks

    # With the default C2 configuration (the metric's N=384 block) the other GPU
    # configurations are timed in the same run: C3 (the north-star 48-block trunk at N=768),
    # C4 (the diffusion transformer) and C5 (the N=1536 block).
    extra = {}
    if args.config == "C4" and not args.no_cached:
        extra["cached_forward_ms"] = round(time_cached_diffusion(res["step"], args.steps, max(1, args.warmup)), 4)
        log(f"C4 with the input cache: {extra['cached_forward_ms']} ms per forward")
    subs = {}
    if args.config == "C2":
        for name, skip in (("C3", args.no_c3), ("C4", args.no_c4), ("C5", args.no_c5)):
            if skip:
                continue
            steps, warmup = DEFAULT_STEPS[name]
            r = run_config(name, steps, warmup, device, graph=args.graph, precondition_s=args.precondition_s)
            if name == "C4":
                sub = {"ms_per_forward": round(r["ms_step"], 4)}
                if not args.no_cached:
                    sub["cached_forward_ms"] = round(time_cached_diffusion(r["step"], steps, warmup), 4)
                    log(f"C4 with the input cache: {sub['cached_forward_ms']} ms per forward")
            else:
                sub = {"ms_per_block": round(r["ms_step"] / r["blocks"], 4)}
                if name == "C3":
                    sub["ms_per_trunk"] = round(r["ms_step"], 3)
            sub.update(steps=steps, warmup=warmup, config=r["workload"], roofline=r["roofline"],
                       kernels=r["kernels"])
            subs[name.lower()] = sub
            del r
            torch.cuda.empty_cache()

    base = None
    if args.config == "T768":
        log("cpu baseline: not measured for the template block")
    elif not args.no_cpu_baseline:
        log("cpu baseline (restatements on host cores)")
        base = cpu_baseline(args.config)
        log(f"cpu baseline: {base}")
        for key, sub in subs.items():
            sub["cpu_baseline"] = cpu_baseline(key.upper())

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
        "config": dict(res["workload"], launch="hip graph replay" if args.graph else "eager",
                       clock_preconditioning_s=args.precondition_s),
        "roofline": res["roofline"], "cpu_baseline": base, "kernels": res["kernels"], **subs, **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
