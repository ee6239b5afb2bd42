"""GridSelfAttention (triangle attention, starting/ending node) with the reference's
constructor, parameter names and call signature (``xfold/nn/attention.py:21-105``),
running on the HIP backend."""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ..fastnn import LayerNorm
from ..fastnn import config as fastnn_config
from ..fastnn import native_hip as nh

_GRID_WEIGHTS = ("pair_bias_projection", "q_projection", "k_projection", "v_projection",
                 "gating_query", "output_projection")


def grid_self_attention_hip(module: nn.Module, pair: torch.Tensor, mask: Optional[torch.Tensor],
                            accumulate_into: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``GridSelfAttention.forward`` (``xfold/nn/attention.py:80-105``): bias from the
    normalised, un-transposed pair; ending node (``transpose=True``) attends along the
    first axis with the mask unchanged; the result is in pair layout."""
    nh.check_gpu_inference(pair, mask, *module.parameters())
    dtype = nh.compute_dtype(pair, *(getattr(module, n).weight for n in _GRID_WEIGHTS))
    if pair.dim() != 3 or pair.shape[0] != pair.shape[1] or pair.shape[2] != module.c_pair:
        raise ValueError("GridSelfAttention expects pair [N, N, c_pair].")
    n, c = pair.shape[0], pair.shape[2]
    heads = module.num_head
    pair_c = pair.contiguous()
    mask_t, mask_code = nh.mask_arg(mask, (n, n)) if mask is not None else (None, nh.BOOL)
    w = {name: nh.linear_weight(module, name, dtype) for name in _GRID_WEIGHTS}
    norm = module.act_norm
    nw = nh.fp32_param(module, "norm_w", norm.weight)
    nb = nh.fp32_param(module, "norm_b", norm.bias)
    if accumulate_into is not None:
        out, accumulate = accumulate_into, 1
        if not out.is_contiguous() or out.shape != pair.shape:
            raise ValueError("accumulate_into must be a contiguous tensor shaped like pair")
    else:
        out, accumulate = torch.empty((n, n, c), dtype=dtype, device=pair.device), 0
    lib = nh.load_library()
    ws = nh.workspace(lib.xfh_grid_self_attention_workspace_size(n, c, heads, nh.dtype_code(dtype)),
                      pair.device)
    nh.call("xfh_grid_self_attention", nh.ptr(pair_c), nh.dtype_code(pair.dtype), nh.ptr(mask_t),
            mask_code, n, c, heads, int(bool(module.transpose)), nh.ptr(nw), nh.ptr(nb),
            float(norm.eps), *(nh.ptr(w[name]) for name in _GRID_WEIGHTS), nh.dtype_code(dtype),
            nh.ptr(out), nh.dtype_code(out.dtype), accumulate, nh.ptr(ws), ws.numel(),
            nh.stream_of(pair.device))
    return out


class GridSelfAttention(nn.Module):
    def __init__(self, c_pair: int = 128, num_head: int = 4, transpose: bool = False):
        super().__init__()
        self.c_pair = c_pair
        self.num_head = num_head
        self.qkv_dim = c_pair // num_head
        self.transpose = transpose
        self.act_norm = LayerNorm(c_pair)
        self.pair_bias_projection = nn.Linear(c_pair, num_head, bias=False)
        self.q_projection = nn.Linear(c_pair, c_pair, bias=False)
        self.k_projection = nn.Linear(c_pair, c_pair, bias=False)
        self.v_projection = nn.Linear(c_pair, c_pair, bias=False)
        self.gating_query = nn.Linear(c_pair, c_pair, bias=False)
        self.output_projection = nn.Linear(c_pair, c_pair, bias=False)

    def forward(self, pair: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        if fastnn_config.dot_product_attention_implementation == fastnn_config.HIP:
            return grid_self_attention_hip(self, pair, mask)
        raise ValueError("Unknown dot_product_attention_implementation for xfold_cpu_amd: "
                         f"{fastnn_config.dot_product_attention_implementation!r} (only 'hip')")
