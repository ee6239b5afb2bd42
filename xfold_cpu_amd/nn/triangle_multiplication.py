"""TriangleMultiplication with the reference's constructor, parameter names and call
signature (``xfold/nn/triangle_multiplication.py:21-46``), running on the HIP backend.

:func:`triangle_multiplication_hip` takes any module that carries the reference's
parameters (this class or the reference's own), so the reference can call it from a
``'hip'`` branch of its ``forward`` without changing checkpoints.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ..fastnn import LayerNorm
from ..fastnn import config as fastnn_config
from ..fastnn import native_hip as nh


def triangle_multiplication_hip(module: nn.Module, pair: torch.Tensor, mask: Optional[torch.Tensor],
                                accumulate_into: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Update of ``xfold/nn/triangle_multiplication.py:71-105`` (or ``pair += update`` in
    place when ``accumulate_into`` is the contiguous pair tensor itself)."""
    names = ("projection", "gate", "output_projection", "gating_linear")
    nh.check_gpu_inference(pair, mask)
    nh.check_module(module)
    dtype = nh.compute_dtype(pair, *(getattr(module, n).weight for n in names))
    if pair.dim() != 3 or pair.shape[0] != pair.shape[1] or pair.shape[2] != module.c_pair:
        raise ValueError("TriangleMultiplication expects pair [N, N, c_pair].")
    n, c = pair.shape[0], pair.shape[2]
    outgoing = module.equation == "cik,cjk->cij"
    pair_c = pair.contiguous()
    mask_t, mask_code = nh.mask_arg(mask, (n, n))
    w = {name: nh.linear_weight(module, name, dtype) for name in names}
    ln_in, ln_c = module.left_norm_input, module.center_norm
    lw = nh.fp32_param(module, "left_w", ln_in.weight)
    lb = nh.fp32_param(module, "left_b", ln_in.bias)
    cw = nh.fp32_param(module, "center_w", ln_c.weight)
    cb = nh.fp32_param(module, "center_b", ln_c.bias)
    if accumulate_into is not None:
        out, accumulate = accumulate_into, 1
        if not out.is_contiguous() or out.shape != pair.shape:
            raise ValueError("accumulate_into must be a contiguous tensor shaped like pair")
    else:
        out, accumulate = torch.empty((n, n, c), dtype=dtype, device=pair.device), 0
    lib = nh.load_library()
    ws = nh.workspace(lib.xfh_triangle_multiplication_workspace_size(n, c, nh.dtype_code(dtype)),
                      pair.device)
    nh.call("xfh_triangle_multiplication", nh.ptr(pair_c), nh.dtype_code(pair.dtype), nh.ptr(mask_t),
            mask_code, n, c, int(outgoing), nh.ptr(lw), nh.ptr(lb), float(ln_in.eps),
            nh.ptr(w["projection"]), nh.ptr(w["gate"]), nh.ptr(cw), nh.ptr(cb), float(ln_c.eps),
            nh.ptr(w["output_projection"]), nh.ptr(w["gating_linear"]), nh.dtype_code(dtype),
            nh.ptr(out), nh.dtype_code(out.dtype), accumulate, nh.ptr(ws), ws.numel(),
            nh.stream_of(pair.device))
    return out


class TriangleMultiplication(nn.Module):
    def __init__(self, c_pair: int = 128, _outgoing: bool = True) -> None:
        super().__init__()
        self.c_pair = c_pair
        self.left_norm_input = LayerNorm(c_pair)
        self.projection = nn.Linear(c_pair, 2 * c_pair, bias=False)
        self.gate = nn.Linear(c_pair, 2 * c_pair, bias=False)
        self.center_norm = LayerNorm(c_pair)
        self.output_projection = nn.Linear(c_pair, c_pair, bias=False)
        self.gating_linear = nn.Linear(c_pair, c_pair, bias=False)
        self.equation = "cik,cjk->cij" if _outgoing else "ckj,cki->cij"

    def forward(self, pair: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        if fastnn_config.triangle_multiplication_implementation == fastnn_config.HIP:
            return triangle_multiplication_hip(self, pair, mask)
        raise ValueError("Unknown triangle_multiplication_implementation for xfold_cpu_amd: "
                         f"{fastnn_config.triangle_multiplication_implementation!r} (only 'hip')")
