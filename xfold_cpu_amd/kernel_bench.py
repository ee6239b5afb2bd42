"""Per-kernel rates of the hot operators on one GPU, against MI355X peaks (HBM 8 TB/s, bf16
dense MFMA 2.5 PFLOP/s).

    python -m xfold_cpu_amd.kernel_bench [--n 768] [--reps 20] [--vendor]

Each operator runs on synthetic bf16 inputs of the Pairformer shapes (pair [N, N, 128]) with
the library's own HIP-event timing (``xfh_set_kernel_timing``) on, so every figure is the
average duration of that kernel's launches on its stream. Bytes are the algorithmic HBM bytes
of one launch (each input read once, each output written once); FLOPs count multiply-adds
as two. One JSON line per kernel.

``--vendor`` adds reference points from the ROCm libraries behind torch at the same shapes,
timed with HIP events around the call: hipBLASLt's batched GEMM on the triangle
contraction's 128 per-channel products, torch's ``scaled_dot_product_attention`` on the
triangle attention's shape with and without its additive bias, a square 8192^3 bf16 GEMM
(what a library GEMM reaches of the MFMA peak on this device), and a 2 GiB device-to-device
copy and elementwise negation (what streaming kernels reach of the HBM peak). They are comparisons, not part of
the backend; the last two are the measured peaks the kernels' fractions can also be read
against.
"""

from __future__ import annotations

import argparse
import json

import torch

from . import nn as hnn
from .fastnn import native_hip as nh
from .fastnn import ops
from .synthetic import init_module_

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0


def pair_kernel_work(n: int, c: int = 128, heads: int = 4, head_dim: int = 32, bias_heads: int = 16):
    """Algorithmic work of one launch of each pair-stack kernel at N tokens: {timer name:
    (kernel, GB or None, GFLOP or None)}. Bytes count each input read once and each output
    written once (bf16 pair, fp32 attention bias); FLOPs count multiply-adds as two."""
    rows = n * n
    npad = (n + 63) // 64 * 64
    gb_pair = rows * c * 2 / 1e9                  # one bf16 pass over the pair
    return {
        "transition": ("transition_kernel", 2 * gb_pair, 2 * rows * (c * 8 * c + 4 * c * c) / 1e9),
        "trimul_project": ("trimul_project_kernel", 3 * gb_pair, None),
        "trimul_contract": ("contraction_kernel", 3 * gb_pair, 2 * c * n ** 3 / 1e9),
        "trimul_output": ("trimul_output_kernel", 3 * gb_pair, None),
        "grid_project": ("grid_project_kernel",
                         gb_pair + (rows * c + 2 * n * heads * npad * head_dim) * 2 / 1e9 + heads * n * npad * 4 / 1e9,
                         None),
        "grid_attention": ("grid_attention_kernel", None, 4 * n * heads * n * n * head_dim / 1e9),
        "grid_output": ("grid_output_kernel", 3 * gb_pair, None),
        "pair_bias": ("pair_bias_kernel", gb_pair + bias_heads * n * npad * 4 / 1e9, None),
    }


def rates(ms, gbytes=None, gflop=None):
    """HBM and MFMA rates of one launch of `ms` milliseconds against the MI355X peaks."""
    rec = {}
    if gbytes is not None:
        rate = gbytes / ms                        # GB per ms = TB/s
        rec.update(bytes_per_launch=gbytes * 1e9, hbm_tbs=round(rate, 3),
                   hbm_frac=round(rate * 1e3 / HBM_PEAK_GBS, 3))
    if gflop is not None:
        tf = gflop / ms                           # GFLOP per ms = TFLOP/s
        rec.update(flops_per_launch=gflop * 1e9, tflops=round(tf, 1), mfma_frac=round(tf / MFMA_PEAK_TFLOPS, 3))
    return rec


def _timed(names, fn, reps):
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    for name in names:
        nh.kernel_timing_read(name)
    nh.set_kernel_timing(True)
    try:
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
    finally:
        nh.set_kernel_timing(False)
    out = {}
    for name in names:
        total_ms, launches = nh.kernel_timing_read(name)
        out[name] = (total_ms / launches if launches else float("nan"), launches)
    return out


def _line(kernel, workload, ms, launches, gbytes=None, gflop=None):
    rec = {"kernel": kernel, "workload": workload, "avg_us": round(ms * 1e3, 2), "launches": launches}
    rec.update(rates(ms, gbytes, gflop))
    print(json.dumps(rec), flush=True)


def _event_ms(fn, reps):
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps


def vendor_points(n: int, reps: int, dev: torch.device, c: int = 128, heads: int = 4, d: int = 32):
    """Library kernels at this path's shapes (comparisons only)."""
    g = torch.Generator(device=dev).manual_seed(0)
    left = torch.randn(c, n, n, device=dev, generator=g).bfloat16()
    right_t = torch.randn(c, n, n, device=dev, generator=g).bfloat16()      # [k][j]: contiguous operand
    prod = torch.empty(c, n, n, device=dev, dtype=torch.bfloat16)
    ms = _event_ms(lambda: torch.bmm(left, right_t, out=prod), reps)
    _line("vendor: torch.bmm (hipBLASLt)", f"{c} products {n}^3 bf16 (the triangle contraction)", ms, reps,
          gflop=2 * c * n ** 3 / 1e9)
    del left, right_t, prod
    q, k, v = (torch.randn(n, heads, n, d, device=dev, generator=g).bfloat16() for _ in range(3))
    bias = torch.randn(1, heads, n, n, device=dev, generator=g).bfloat16().expand(n, heads, n, n)
    flop = 4 * n * heads * n * n * d / 1e9
    sdpa = torch.nn.functional.scaled_dot_product_attention
    ms = _event_ms(lambda: sdpa(q, k, v, attn_mask=bias), reps)
    _line("vendor: scaled_dot_product_attention + bias", f"B={n} H={heads} Q=K={n} D={d} bf16", ms, reps, gflop=flop)
    ms = _event_ms(lambda: sdpa(q, k, v), reps)
    _line("vendor: scaled_dot_product_attention", f"B={n} H={heads} Q=K={n} D={d} bf16, no bias", ms, reps,
          gflop=flop)
    del q, k, v, bias
    big = 8192
    a = torch.randn(big, big, device=dev, generator=g).bfloat16()
    b = torch.randn(big, big, device=dev, generator=g).bfloat16()
    out = torch.empty(big, big, device=dev, dtype=torch.bfloat16)
    ms = _event_ms(lambda: torch.mm(a, b, out=out), max(reps // 2, 3))
    _line("vendor: torch.mm (hipBLASLt)", f"{big}^3 bf16", ms, reps, gflop=2 * big ** 3 / 1e9)
    del a, b, out
    src = torch.ones(1 << 29, device=dev, dtype=torch.float32)
    dst = torch.empty_like(src)
    ms = _event_ms(lambda: dst.copy_(src), max(reps // 2, 3))
    _line("vendor: Tensor.copy_", "2 GiB device to device (read + write)", ms, reps, gbytes=2 * 4 * src.numel() / 1e9)
    ms = _event_ms(lambda: torch.neg(src, out=dst), max(reps // 2, 3))
    _line("vendor: torch.neg", "2 GiB fp32 elementwise (read + write)", ms, reps, gbytes=2 * 4 * src.numel() / 1e9)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--n", type=int, default=768)
    p.add_argument("--reps", type=int, default=20)
    p.add_argument("--vendor", action="store_true", help="add the library reference points")
    args = p.parse_args(argv)
    n, c = args.n, 128
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    rows = n * n
    pair = torch.randn(n, n, c, device=dev).bfloat16()
    mask = torch.ones(n, n, device=dev)
    gb_pair = rows * c * 2 / 1e9                  # one bf16 pass over the pair
    work = pair_kernel_work(n, c)
    with torch.inference_mode():
        # LayerNorm over the pair rows, bf16 -> bf16 and fp32 -> bf16.
        w, b = torch.ones(c, device=dev), torch.zeros(c, device=dev)
        r = _timed(["layer_norm"], lambda: ops.layer_norm(pair, (c,), w, b, 1e-5, out_dtype=torch.bfloat16), args.reps)
        _line("ln_rows_vec", f"LayerNorm [{rows}, {c}] bf16 -> bf16", *r["layer_norm"], gbytes=2 * gb_pair)
        pair32 = pair.float()
        r = _timed(["layer_norm"], lambda: ops.layer_norm(pair32, (c,), w, b, 1e-5, out_dtype=torch.bfloat16), args.reps)
        _line("ln_rows_vec", f"LayerNorm [{rows}, {c}] fp32 -> bf16", *r["layer_norm"], gbytes=3 * gb_pair)
        del pair32
        with torch.amp.autocast("cuda", dtype=torch.bfloat16):
            # Pair transition (GLU 128 -> 2 x 512 -> 128), added into the pair in place.
            tr = init_module_(hnn.Transition(c_x=c, num_intermediate_factor=4), seed=1).to(dev).eval()
            r = _timed(["transition"], lambda: hnn.transition_hip(tr, pair, accumulate_into=pair), args.reps)
            _line("transition_kernel", f"pair transition N={n}", *r["transition"], *work["transition"][1:])
            # Triangle multiplication (outgoing): projection, contraction, output.
            tm = init_module_(hnn.TriangleMultiplication(c_pair=c, _outgoing=True), seed=2).to(dev).eval()
            names = ["trimul_project", "trimul_contract", "trimul_output"]
            r = _timed(names, lambda: hnn.triangle_multiplication_hip(tm, pair, mask, accumulate_into=pair),
                       args.reps)
            _line("trimul_project_kernel", f"TriMul projection N={n}", *r["trimul_project"], *work["trimul_project"][1:])
            _line("contraction_kernel", f"TriMul contraction N={n}", *r["trimul_contract"], *work["trimul_contract"][1:])
            _line("trimul_output_kernel", f"TriMul output N={n}", *r["trimul_output"], *work["trimul_output"][1:])
            # Triangle attention (starting node): projection, attention core, output.
            ga = init_module_(hnn.GridSelfAttention(c_pair=c, num_head=4, transpose=False), seed=3).to(dev).eval()
            names = ["grid_project", "grid_attention", "grid_output"]
            r = _timed(names, lambda: hnn.grid_self_attention_hip(ga, pair, mask, accumulate_into=pair), args.reps)
            _line("grid_project_kernel", f"TriAtt projection N={n}", *r["grid_project"], *work["grid_project"][1:])
            _line("grid_attention_kernel", f"TriAtt core N={n}, 4 heads x 32", *r["grid_attention"],
                  *work["grid_attention"][1:])
            _line("grid_output_kernel", f"TriAtt output N={n}", *r["grid_output"], *work["grid_output"][1:])
            # Pair-logits attention bias (single-track attention, 16 heads).
            wl = (torch.randn(16, c, device=dev) / c ** 0.5).bfloat16()
            r = _timed(["pair_bias"], lambda: ops.pair_attention_bias(pair, w, b, 1e-5, wl), args.reps)
            _line("pair_bias_kernel", f"pair logits N={n}, 16 heads", *r["pair_bias"], *work["pair_bias"][1:])
            # The pair transition with the single track's pair logits in its epilogue (one
            # launch; the logits add their fp32 writes to the transition's bytes).
            blk = init_module_(hnn.PairformerBlock(n_heads=16, c_pair=c, c_single=384, n_heads_pair=4,
                                                   with_single=True), seed=4).to(dev).eval()
            from .nn import pairformer
            r = _timed(["transition"], lambda: pairformer._transition_with_logits_hip(blk, pair), args.reps)
            npad = (n + 63) // 64 * 64
            _line("transition_kernel + pair logits", f"pair transition with 16-head logits N={n}", *r["transition"],
                  work["transition"][1] + 16 * n * npad * 4 / 1e9, work["transition"][2] + 2 * rows * c * 16 / 1e9)
    if args.vendor:
        del pair, mask
        with torch.inference_mode():
            vendor_points(n, args.reps, dev)


if __name__ == "__main__":
    main()
