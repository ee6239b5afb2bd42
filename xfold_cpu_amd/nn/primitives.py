"""Transition (LN -> GLU -> Linear) with the reference's constructor and parameter names
(``xfold/nn/primitives.py:20-37``), running on the HIP backend."""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ..fastnn import LayerNorm
from ..fastnn import config as fastnn_config
from ..fastnn import native_hip as nh


def transition_hip(module: nn.Module, x: torch.Tensor,
                   accumulate_into: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``transition2(GLU(LN(x), transition1.weight.T))`` (``xfold/nn/primitives.py:33-37``)."""
    nh.check_gpu_inference(x, *module.parameters())
    dtype = nh.compute_dtype(x, module.transition1.weight, module.transition2.weight)
    c = x.shape[-1]
    f = module.transition2.weight.shape[1]
    if module.transition1.weight.shape != (2 * f, c):
        raise ValueError("Transition weights do not match the input width.")
    x_c = x.contiguous()
    rows = x_c.numel() // c
    w1 = nh.linear_weight(module, "transition1", dtype, "glu")
    w2 = nh.linear_weight(module, "transition2", dtype)
    norm = module.input_layer_norm
    nw = nh.fp32_param(module, "norm_w", norm.weight)
    nb = nh.fp32_param(module, "norm_b", norm.bias)
    if accumulate_into is not None:
        out, accumulate = accumulate_into, 1
        if not out.is_contiguous() or out.shape != x.shape:
            raise ValueError("accumulate_into must be a contiguous tensor shaped like x")
    else:
        out, accumulate = torch.empty(x.shape, dtype=dtype, device=x.device), 0
    lib = nh.load_library()
    ws = nh.workspace(lib.xfh_transition_workspace_size(rows, c, f, nh.dtype_code(dtype)), x.device)
    nh.call("xfh_transition", nh.ptr(x_c), nh.dtype_code(x.dtype), rows, c, f, nh.ptr(nw), nh.ptr(nb),
            float(norm.eps), nh.ptr(w1), nh.ptr(w2), nh.dtype_code(dtype), nh.ptr(out),
            nh.dtype_code(out.dtype), accumulate, nh.ptr(ws), ws.numel(), nh.stream_of(x.device))
    return out


class Transition(nn.Module):
    def __init__(self, c_x: int, num_intermediate_factor: int = 4) -> None:
        super().__init__()
        self.num_intermediate_factor = num_intermediate_factor
        self.c_in = c_x
        self.input_layer_norm = LayerNorm(c_x)
        self.transition1 = nn.Linear(c_x, num_intermediate_factor * c_x * 2, bias=False)
        self.transition2 = nn.Linear(num_intermediate_factor * c_x, c_x, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if fastnn_config.gated_linear_unit_implementation == fastnn_config.HIP:
            return transition_hip(self, x)
        raise ValueError("Unknown gated_linear_unit_implementation for xfold_cpu_amd: "
                         f"{fastnn_config.gated_linear_unit_implementation!r} (only 'hip')")
