"""GridSelfAttention (triangle attention, starting/ending node) and MSAAttention with the
reference's constructors, parameter names and call signatures (``xfold/nn/attention.py:21-144``),
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
    nh.check_gpu_inference(pair, mask)
    nh.check_module(module)
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


_MSA_WEIGHTS = ("pair_logits", "v_projection", "gating_query", "output_projection")


def msa_attention_hip(module: nn.Module, msa: torch.Tensor, msa_mask: Optional[torch.Tensor],
                      pair: torch.Tensor, accumulate_into: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``MSAAttention.forward`` (``xfold/nn/attention.py:126-144``): msa [S, N, c_msa],
    msa_mask [S, N], pair [N, N, c_pair] -> [S, N, c_msa]. The attention weights come from
    the pair alone (with the key term ``1e9 * (max_s mask - 1)``) and are shared by every
    MSA row."""
    nh.check_gpu_inference(msa, msa_mask, pair)
    nh.check_module(module)
    dtype = nh.compute_dtype(msa, *(getattr(module, n).weight for n in _MSA_WEIGHTS))
    if msa.dim() != 3 or msa.shape[-1] != module.c_msa:
        raise ValueError("MSAAttention expects msa [S, N, c_msa].")
    rows, n, c_msa = msa.shape
    if tuple(pair.shape) != (n, n, module.c_pair):
        raise ValueError("MSAAttention expects pair [N, N, c_pair] matching msa.")
    if pair.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("The 'hip' backend supports FP32/BF16 only.")
    msa_c, pair_c = msa.contiguous(), pair.contiguous()
    mask_t, mask_code = nh.mask_arg(msa_mask, (rows, n)) if msa_mask is not None else (None, nh.BOOL)
    w = {name: nh.linear_weight(module, name, dtype) for name in _MSA_WEIGHTS}
    act_norm, pair_norm = module.act_norm, module.pair_norm
    if accumulate_into is not None:
        out, accumulate = accumulate_into, 1
        if not out.is_contiguous() or out.shape != msa.shape:
            raise ValueError("accumulate_into must be a contiguous tensor shaped like msa")
    else:
        out, accumulate = torch.empty((rows, n, c_msa), dtype=dtype, device=msa.device), 0
    lib = nh.load_library()
    ws = nh.workspace(lib.xfh_msa_attention_workspace_size(rows, n, c_msa, module.c_pair, module.num_head,
                                                           nh.dtype_code(dtype)), msa.device)
    nh.call("xfh_msa_attention", nh.ptr(msa_c), nh.dtype_code(msa.dtype), nh.ptr(mask_t), mask_code,
            nh.ptr(pair_c), nh.dtype_code(pair.dtype), rows, n, c_msa, module.c_pair, module.num_head,
            nh.ptr(nh.fp32_param(module, "act_norm_w", act_norm.weight)),
            nh.ptr(nh.fp32_param(module, "act_norm_b", act_norm.bias)), float(act_norm.eps),
            nh.ptr(nh.fp32_param(module, "pair_norm_w", pair_norm.weight)),
            nh.ptr(nh.fp32_param(module, "pair_norm_b", pair_norm.bias)), float(pair_norm.eps),
            *(nh.ptr(w[name]) for name in _MSA_WEIGHTS), nh.dtype_code(dtype), nh.ptr(out),
            nh.dtype_code(out.dtype), accumulate, nh.ptr(ws), ws.numel(), nh.stream_of(msa.device))
    return out


class MSAAttention(nn.Module):
    def __init__(self, c_msa: int = 64, c_pair: int = 128, num_head: int = 8):
        super().__init__()
        self.c_msa = c_msa
        self.c_pair = c_pair
        self.num_head = num_head
        self.value_dim = c_msa // num_head
        self.act_norm = LayerNorm(c_msa)
        self.pair_norm = LayerNorm(c_pair)
        self.pair_logits = nn.Linear(c_pair, num_head, bias=False)
        self.v_projection = nn.Linear(c_msa, num_head * self.value_dim, bias=False)
        self.gating_query = nn.Linear(c_msa, c_msa, bias=False)
        self.output_projection = nn.Linear(c_msa, c_msa, bias=False)

    def forward(self, msa: torch.Tensor, msa_mask: torch.Tensor, pair: torch.Tensor) -> torch.Tensor:
        if fastnn_config.layer_norm_implementation == fastnn_config.HIP:
            return msa_attention_hip(self, msa, msa_mask, pair)
        raise ValueError("Unknown layer_norm_implementation for xfold_cpu_amd: "
                         f"{fastnn_config.layer_norm_implementation!r} (only 'hip')")
