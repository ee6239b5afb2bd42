"""Transition (LN -> GLU -> Linear) and OuterProductMean with the reference's constructors
and parameter names (``xfold/nn/primitives.py:20-72``), running on the HIP backend."""

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
    nh.check_gpu_inference(x)
    nh.check_module(module)
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


def _opm_output_weight(module: nn.Module, dtype: torch.dtype) -> torch.Tensor:
    """``output_w`` [c, e, f] as the GEMM weight [f, c * e] in ``dtype`` (made once per
    parameter version)."""
    def build(w):
        c, e, f = w.shape
        return w.detach().permute(2, 0, 1).reshape(f, c * e).to(dtype).contiguous()
    return nh.derived_weight(module, f"opm_output_w:{dtype}", [module.output_w], build)


def outer_product_mean_hip(module: nn.Module, msa: torch.Tensor, mask: torch.Tensor,
                           accumulate_into: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``OuterProductMean.forward`` (``xfold/nn/primitives.py:58-72``): msa [S, N, c_msa],
    mask [S, N] -> [N, N, num_output_channel]; the left x right outer product summed over
    the S sequences, projected by ``output_w``, plus ``output_b``, divided by
    ``epsilon + sum_s mask[s, i] mask[s, j]``."""
    nh.check_gpu_inference(msa, mask)
    nh.check_module(module)
    dtype = nh.compute_dtype(msa, module.left_projection.weight, module.right_projection.weight)
    if msa.dim() != 3 or msa.shape[-1] != module.c_msa:
        raise ValueError("OuterProductMean expects msa [S, N, c_msa].")
    rows, n, c_msa = msa.shape
    co, c_out = module.num_outer_channel, module.num_output_channel
    msa_c = msa.contiguous()
    mask_t, mask_code = nh.mask_arg(mask, (rows, n)) if mask is not None else (None, nh.BOOL)
    proj = nh.fused_linear_weight(module, ("left_projection", "right_projection"), dtype)
    w_out = _opm_output_weight(module, dtype)
    b_out = nh.fp32_param(module, "output_b", module.output_b)
    norm = module.layer_norm_input
    nw = nh.fp32_param(module, "norm_w", norm.weight)
    nb = nh.fp32_param(module, "norm_b", norm.bias)
    if accumulate_into is not None:
        out, accumulate = accumulate_into, 1
        if not out.is_contiguous() or tuple(out.shape) != (n, n, c_out):
            raise ValueError("accumulate_into must be a contiguous [N, N, num_output_channel] tensor")
    else:
        out, accumulate = torch.empty((n, n, c_out), dtype=dtype, device=msa.device), 0
    lib = nh.load_library()
    ws = nh.workspace(lib.xfh_outer_product_mean_workspace_size(rows, n, c_msa, co, nh.dtype_code(dtype)),
                      msa.device)
    nh.call("xfh_outer_product_mean", nh.ptr(msa_c), nh.dtype_code(msa.dtype), nh.ptr(mask_t), mask_code,
            rows, n, c_msa, co, c_out, nh.ptr(nw), nh.ptr(nb), float(norm.eps), nh.ptr(proj), nh.ptr(w_out),
            nh.ptr(b_out), float(module.epsilon), nh.dtype_code(dtype), nh.ptr(out), nh.dtype_code(out.dtype),
            accumulate, nh.ptr(ws), ws.numel(), nh.stream_of(msa.device))
    return out


class OuterProductMean(nn.Module):
    def __init__(self, c_msa: int = 64, num_output_channel: int = 128, num_outer_channel: int = 32) -> None:
        super().__init__()
        self.c_msa = c_msa
        self.num_outer_channel = num_outer_channel
        self.num_output_channel = num_output_channel
        self.epsilon = 1e-3
        self.layer_norm_input = LayerNorm(c_msa)
        self.left_projection = nn.Linear(c_msa, num_outer_channel, bias=False)
        self.right_projection = nn.Linear(c_msa, num_outer_channel, bias=False)
        self.output_w = nn.Parameter(torch.randn(num_outer_channel, num_outer_channel, num_output_channel))
        self.output_b = nn.Parameter(torch.randn(num_output_channel))

    def forward(self, msa: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        if fastnn_config.layer_norm_implementation == fastnn_config.HIP:
            return outer_product_mean_hip(self, msa, mask)
        raise ValueError("Unknown layer_norm_implementation for xfold_cpu_amd: "
                         f"{fastnn_config.layer_norm_implementation!r} (only 'hip')")
