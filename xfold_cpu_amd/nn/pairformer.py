"""PairformerBlock and EvoformerBlock with the reference's constructors, submodule names and
call signatures (``xfold/nn/pairformer.py:26-156``), running on the HIP backend.

The block applies its five pair updates in place, each op's final kernel adding its
result straight into ``pair`` (the residual ``pair += op(pair)`` of ``pairformer.py:96-100``
without a separate update tensor), then the single track (``pairformer.py:102-113``).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ..fastnn import LayerNorm
from ..fastnn import config as fastnn_config
from ..fastnn import native_hip as nh
from ..fastnn import ops
from .attention import GridSelfAttention, MSAAttention, grid_self_attention_hip, msa_attention_hip
from .diffusion_transformer import SelfAttention, self_attention_hip
from .primitives import OuterProductMean, Transition, outer_product_mean_hip, transition_hip
from .triangle_multiplication import TriangleMultiplication, triangle_multiplication_hip


def pair_logits_hip(block: nn.Module, pair: torch.Tensor, dtype: torch.dtype):
    """``Linear(LN(pair)).permute(2, 0, 1)`` (``pairformer.py:103-106``): with bf16 compute,
    128 pair channels and at most ``attention_max_keys()`` tokens one kernel writes it as the
    attention's packed bias (:class:`ops.PackedBias`), else a [H, N, N] view."""
    norm = block.single_pair_logits_norm
    proj = block.single_pair_logits_projection
    if dtype == torch.bfloat16 and pair.shape[-1] == 128 and proj.weight.shape[0] <= 384 \
            and tuple(norm.normalized_shape) == (128,) and pair.shape[0] <= nh.attention_max_keys():
        w = nh.linear_weight(block, "single_pair_logits_projection", dtype)
        return ops.PackedBias(ops.pair_attention_bias(pair, norm.weight, norm.bias, norm.eps, w, owner=norm))
    normed = ops.layer_norm(pair, norm.normalized_shape, norm.weight, norm.bias, norm.eps,
                            out_dtype=dtype, owner=norm)
    logits = ops.linear(normed, nh.linear_weight(block, "single_pair_logits_projection", dtype), None, dtype)
    return logits.permute(2, 0, 1)


# The single-track block's pair transition and pair logits in one kernel (when the shapes
# allow it); False runs them as two kernels, with the same results bit for bit.
FUSE_TRANSITION_AND_LOGITS = True


def _transition_with_logits_hip(block: nn.Module, pair: torch.Tensor) -> Optional[ops.PackedBias]:
    """``pair += pair_transition(pair)`` and then the pair logits of the updated pair
    (``pairformer.py:100``, ``:103-106``) in one kernel, whose epilogue computes the logits
    from the values it stores: bf16 pair [N, N, 128], hidden 512, at most 16 heads. None
    (nothing done) for other shapes."""
    tr, norm = block.pair_transition, block.single_pair_logits_norm
    proj = block.single_pair_logits_projection
    n, c = pair.shape[0], pair.shape[-1]
    if (pair.dtype != torch.bfloat16 or pair.dim() != 3 or pair.shape[1] != n or c != 128
            or tr.transition2.weight.shape != (c, 512) or tr.transition1.weight.shape != (1024, c)
            or tuple(norm.normalized_shape) != (c,) or tuple(tr.input_layer_norm.normalized_shape) != (c,)
            or proj.weight.shape[0] > 16 or n > nh.attention_max_keys()
            or nh.compute_dtype(pair, tr.transition1.weight, tr.transition2.weight, proj.weight) != torch.bfloat16):
        return None
    nh.check_gpu_inference(pair)
    nh.check_module(tr)
    w1 = nh.linear_weight(tr, "transition1", torch.bfloat16, "glu")
    w2 = nh.linear_weight(tr, "transition2", torch.bfloat16)
    nw = nh.fp32_param(tr, "norm_w", tr.input_layer_norm.weight)
    nb = nh.fp32_param(tr, "norm_b", tr.input_layer_norm.bias)
    wb = nh.linear_weight(block, "single_pair_logits_projection", torch.bfloat16)
    bw = nh.fp32_param(norm, "ln_weight", norm.weight)
    bb = nh.fp32_param(norm, "ln_bias", norm.bias)
    heads = wb.shape[0]
    packed = torch.empty((heads, n, (n + 63) // 64 * 64), dtype=torch.float32, device=pair.device)
    nh.call("xfh_transition_pair_bias", nh.ptr(pair), n, c, 512, nh.ptr(nw), nh.ptr(nb),
            float(tr.input_layer_norm.eps), nh.ptr(w1), nh.ptr(w2), nh.ptr(bw), nh.ptr(bb), float(norm.eps),
            nh.ptr(wb.contiguous()), heads, nh.ptr(packed), nh.stream_of(pair.device))
    return ops.PackedBias(packed)


def pairformer_block_hip(block: nn.Module, pair: torch.Tensor, pair_mask: torch.Tensor,
                         single: Optional[torch.Tensor] = None,
                         seq_mask: Optional[torch.Tensor] = None):
    """``PairformerBlock.forward`` (``pairformer.py:77-114``); ``pair`` (and ``single``)
    must be contiguous and are updated in place, as the reference's ``+=`` does."""
    if not pair.is_contiguous() or (single is not None and not single.is_contiguous()):
        raise ValueError("PairformerBlock (hip) updates pair/single in place; pass contiguous tensors")
    if not block.with_single:
        _pair_updates_hip(block, pair, pair_mask)
        return pair
    _pair_updates_hip(block, pair, pair_mask, transition=False)
    logits = _transition_with_logits_hip(block, pair) if FUSE_TRANSITION_AND_LOGITS else None
    if logits is None:
        transition_hip(block.pair_transition, pair, accumulate_into=pair)
        dtype = nh.compute_dtype(pair, block.single_pair_logits_projection.weight)
        logits = pair_logits_hip(block, pair, dtype)
    self_attention_hip(block.single_attention_, single, seq_mask, logits, None, accumulate_into=single)
    transition_hip(block.single_transition, single, accumulate_into=single)
    return pair, single


def _pair_updates_hip(block: nn.Module, pair: torch.Tensor, pair_mask: torch.Tensor,
                      transition: bool = True) -> None:
    triangle_multiplication_hip(block.triangle_multiplication_outgoing, pair, pair_mask, accumulate_into=pair)
    triangle_multiplication_hip(block.triangle_multiplication_incoming, pair, pair_mask, accumulate_into=pair)
    grid_self_attention_hip(block.pair_attention1, pair, pair_mask, accumulate_into=pair)
    grid_self_attention_hip(block.pair_attention2, pair, pair_mask, accumulate_into=pair)
    if transition:
        transition_hip(block.pair_transition, pair, accumulate_into=pair)


def _require_hip_backends() -> None:
    for name in ("layer_norm_implementation", "dot_product_attention_implementation",
                 "gated_linear_unit_implementation", "triangle_multiplication_implementation"):
        if getattr(fastnn_config, name) != fastnn_config.HIP:
            raise ValueError(f"Unknown {name} for xfold_cpu_amd: "
                             f"{getattr(fastnn_config, name)!r} (only 'hip')")


class PairformerBlock(nn.Module):
    def __init__(self, n_heads: int = 16, c_pair: int = 128, c_single: int = 384,
                 c_hidden_mul: int = 128, n_heads_pair: int = 4, num_intermediate_factor: int = 4,
                 with_single: bool = True) -> None:
        super().__init__()
        self.n_heads = n_heads
        self.with_single = with_single
        self.num_intermediate_factor = num_intermediate_factor
        self.triangle_multiplication_outgoing = TriangleMultiplication(c_pair=c_pair, _outgoing=True)
        self.triangle_multiplication_incoming = TriangleMultiplication(c_pair=c_pair, _outgoing=False)
        self.pair_attention1 = GridSelfAttention(c_pair=c_pair, num_head=n_heads_pair, transpose=False)
        self.pair_attention2 = GridSelfAttention(c_pair=c_pair, num_head=n_heads_pair, transpose=True)
        self.pair_transition = Transition(c_x=c_pair, num_intermediate_factor=num_intermediate_factor)
        self.c_single = c_single
        if with_single:
            self.single_pair_logits_norm = LayerNorm(c_pair)
            self.single_pair_logits_projection = nn.Linear(c_pair, n_heads, bias=False)
            self.single_attention_ = SelfAttention(c_x=c_single, num_head=n_heads, use_single_cond=False)
            self.single_transition = Transition(c_x=c_single)

    def forward(self, pair, pair_mask, single=None, seq_mask=None):
        _require_hip_backends()
        return pairformer_block_hip(self, pair, pair_mask, single, seq_mask)


def evoformer_block_hip(block: nn.Module, msa: torch.Tensor, pair: torch.Tensor, msa_mask: torch.Tensor,
                        pair_mask: torch.Tensor):
    """``EvoformerBlock.forward`` (``pairformer.py:139-156``): OuterProductMean into the pair,
    MSA attention (over the updated pair) and transition into the MSA, then the five pair
    updates. ``msa`` and ``pair`` must be contiguous and are updated in place."""
    if not pair.is_contiguous() or not msa.is_contiguous():
        raise ValueError("EvoformerBlock (hip) updates msa/pair in place; pass contiguous tensors")
    outer_product_mean_hip(block.outer_product_mean, msa, msa_mask, accumulate_into=pair)
    msa_attention_hip(block.msa_attention1, msa, msa_mask, pair, accumulate_into=msa)
    transition_hip(block.msa_transition, msa, accumulate_into=msa)
    _pair_updates_hip(block, pair, pair_mask)
    return msa, pair


class EvoformerBlock(nn.Module):
    def __init__(self, c_msa: int = 64, c_pair: int = 128, n_heads_pair: int = 4) -> None:
        super().__init__()
        self.outer_product_mean = OuterProductMean(c_msa=c_msa, num_output_channel=c_pair)
        self.msa_attention1 = MSAAttention(c_msa=c_msa, c_pair=c_pair)
        self.msa_transition = Transition(c_x=c_msa)
        self.triangle_multiplication_outgoing = TriangleMultiplication(c_pair=c_pair, _outgoing=True)
        self.triangle_multiplication_incoming = TriangleMultiplication(c_pair=c_pair, _outgoing=False)
        self.pair_attention1 = GridSelfAttention(c_pair=c_pair, num_head=n_heads_pair, transpose=False)
        self.pair_attention2 = GridSelfAttention(c_pair=c_pair, num_head=n_heads_pair, transpose=True)
        self.pair_transition = Transition(c_x=c_pair)

    def forward(self, msa, pair, msa_mask, pair_mask):
        _require_hip_backends()
        return evoformer_block_hip(self, msa, pair, msa_mask, pair_mask)
