"""CPU restatement of the reference's PyTorch backend for the Pairformer hot path.

Test infrastructure only (see ``oracle/__init__.py``). Every function and module below
restates, in this repository's own code, the op sequence and dtype boundaries of the
reference's ``torch`` implementation, citing the reference file:line it follows. Module
and parameter names are the reference's, so one ``state_dict`` loads into these modules,
into the reference's modules and into ``xfold_cpu_amd.nn``'s HIP modules alike.

All references are paths inside the reference repository (Zhengye-AIsys/xfold_cpu).
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


# ----------------------------------------------------------------------------------------
# fastnn operators
# ----------------------------------------------------------------------------------------

class LayerNorm(nn.Module):
    """``xfold/fastnn/layer_norm.py:14-59`` (torch branch): F.layer_norm over the last dims.

    Parameters are ``weight`` (ones) and ``bias`` (zeros) as in ``reset_parameters``
    (``layer_norm.py:49-53``); ``elementwise_affine=False`` registers neither and
    ``bias=False`` keeps only ``weight`` (``layer_norm.py:33-46``). eps defaults to 1e-5
    (``layer_norm.py:18``).
    """

    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True,
                 bias: bool = True) -> None:
        super().__init__()
        if isinstance(normalized_shape, int):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(self.normalized_shape))
            self.bias = nn.Parameter(torch.zeros(self.normalized_shape)) if bias else None
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.layer_norm(x, self.normalized_shape, self.weight, self.bias, self.eps)


def gated_linear_unit(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``xfold/fastnn/gated_linear_unit.py:103-107``.

    ``weight`` is ``[K, 2F]`` (callers pass ``transition1.weight.T``); the first F output
    columns are the SiLU gate, the last F the value.
    """
    projected = torch.matmul(x, weight)
    gate, value = torch.chunk(projected, 2, dim=-1)
    return F.silu(gate) * value


def _broadcast_key_mask(mask: torch.Tensor) -> torch.Tensor:
    """Mask ranks per ``xfold/fastnn/attention.py:57-61``: 1-D -> [1,1,1,K], 2-D -> [B,1,1,K]."""
    if mask.dim() == 1:
        return mask[None, None, None, :].to(dtype=torch.bool)
    if mask.dim() == 2:
        return mask[:, None, None, :].to(dtype=torch.bool)
    return mask


def _attention_4d(q, k, v, mask, bias):
    """``xfold/fastnn/attention.py:45-66``: scale q, q@k^T, += bias, fill -1e9, softmax, @v."""
    q = q * (q.size(-1) ** -0.5)
    logits = torch.matmul(q, k.transpose(-1, -2))
    if bias is not None:
        logits += bias
    if mask is not None:
        logits.masked_fill_(~_broadcast_key_mask(mask), -1e9)
    probabilities = torch.softmax(logits, dim=-1)
    return torch.matmul(probabilities, v)


def dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          mask: Optional[torch.Tensor] = None,
                          bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``xfold/fastnn/attention.py:69-98`` with the torch body: 3-D inputs gain a batch dim."""
    unbatched = q.dim() == 3
    if unbatched:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    out = _attention_4d(q, k, v, mask, bias)
    return out.squeeze(0) if unbatched else out


def dot_product_attention_chunked(q, k, v, mask=None, bias=None, rows_per_chunk: int = 16):
    """Same semantics as :func:`dot_product_attention` for 4-D inputs, evaluated over
    chunks of the batch dim so the [B, H, Q, K] logits never exist at once.

    Batch rows are independent in ``xfold/fastnn/attention.py:45-66``; a 2-D mask and a
    batch-broadcast bias are sliced along with them. Used for the CPU baseline at large N.
    """
    outs = []
    batches = q.size(0)
    for start in range(0, batches, rows_per_chunk):
        stop = min(batches, start + rows_per_chunk)
        m = mask
        if m is not None and m.dim() == 2:
            m = m[start:stop]
        elif m is not None and m.dim() == 4 and m.size(0) != 1:
            m = m[start:stop]
        b = bias
        if b is not None and b.dim() == 4 and b.size(0) != 1:
            b = b[start:stop]
        outs.append(_attention_4d(q[start:stop], k[start:stop], v[start:stop], m, b))
    return torch.cat(outs, dim=0)


# ----------------------------------------------------------------------------------------
# nn modules
# ----------------------------------------------------------------------------------------

def _heads_first(t: torch.Tensor, num_head: int) -> torch.Tensor:
    """'b n (h d) -> b h n d' (``xfold/nn/attention.py:71-72``) and 'n (h c) -> h n c'."""
    *lead, n, channels = t.shape
    t = t.reshape(*lead, n, num_head, channels // num_head)
    return t.transpose(-3, -2)


def _heads_last(t: torch.Tensor) -> torch.Tensor:
    """'b h n d -> b n (h d)' (``xfold/nn/attention.py:78``) and 'h q c -> q (h c)'."""
    t = t.transpose(-3, -2)
    *lead, n, h, d = t.shape
    return t.reshape(*lead, n, h * d)


class TriangleMultiplication(nn.Module):
    """``xfold/nn/triangle_multiplication.py:21-105`` (``_forward_torch`` at :71-105).

    Outgoing ``'cik,cjk->cij'``, incoming ``'ckj,cki->cij'`` (:34-36). The projection is
    masked, then gated by sigmoid(gate) (:85-90); channel 2k is ``a``, 2k+1 is ``b``
    (:92-95); the output gate uses the normalised input (:81, :102-103). Returns the
    update; the residual is the caller's (``xfold/nn/pairformer.py:96-97``).
    """

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

    def forward(self, pair: torch.Tensor, mask: Optional[torch.Tensor]) -> torch.Tensor:
        normed = self.left_norm_input(pair)
        projected = self.projection(normed).permute(2, 0, 1)
        if mask is not None:
            projected *= mask[None, ...]
        gate = self.gate(normed).permute(2, 0, 1)
        projected *= torch.sigmoid(gate)
        projected = projected.reshape(self.c_pair, 2, *projected.shape[1:])
        left = projected[:, 0]
        right = projected[:, 1]
        contracted = torch.einsum(self.equation, left, right).permute(1, 2, 0)
        update = self.output_projection(self.center_norm(contracted))
        update *= torch.sigmoid(self.gating_linear(normed))
        return update


class GridSelfAttention(nn.Module):
    """``xfold/nn/attention.py:21-105`` (torch path :61-78, forward :80-105).

    The pair bias comes from the normalised, *un-transposed* pair (:89-95); the ending
    node (``transpose=True``) transposes only the attention input/output (:97-103); the
    mask is passed through unchanged.
    """

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

    def forward(self, pair: torch.Tensor, mask: torch.Tensor, attention=None) -> torch.Tensor:
        attention = attention or dot_product_attention
        normed = self.act_norm(pair)
        bias = self.pair_bias_projection(normed).permute(2, 0, 1)
        if self.transpose:
            normed = normed.permute(1, 0, 2)
        q = _heads_first(self.q_projection(normed), self.num_head)
        k = _heads_first(self.k_projection(normed), self.num_head)
        v = _heads_first(self.v_projection(normed), self.num_head)
        weighted = _heads_last(attention(q, k, v, mask=mask, bias=bias))
        weighted *= torch.sigmoid(self.gating_query(normed))
        out = self.output_projection(weighted)
        if self.transpose:
            out = out.permute(1, 0, 2)
        return out


def grid_self_attention_rows(module: "GridSelfAttention", pair: torch.Tensor, mask: torch.Tensor,
                             rows: torch.Tensor, attention=None) -> torch.Tensor:
    """Batch rows ``rows`` of ``GridSelfAttention.forward`` (``xfold/nn/attention.py:80-105``)
    without evaluating the others: the starting node's output pair rows ``out[rows]``, the
    ending node's output pair columns ``out[:, rows]`` returned as ``[len(rows), n, c]``.

    Batch rows are independent once the bias (from the whole normalised pair, :89-95) is
    known: each row's q/k/v/gate come from that row of the (transposed) input (:97-100),
    and its 2-D mask row is ``mask[row]`` (``xfold/fastnn/attention.py:57-61``). Used at
    sizes where evaluating every row on the host would take minutes.
    """
    attention = attention or dot_product_attention
    normed = module.act_norm(pair)
    bias = module.pair_bias_projection(normed).permute(2, 0, 1)
    if module.transpose:
        normed = normed.permute(1, 0, 2)
    x = normed[rows]
    q = _heads_first(module.q_projection(x), module.num_head)
    k = _heads_first(module.k_projection(x), module.num_head)
    v = _heads_first(module.v_projection(x), module.num_head)
    weighted = _heads_last(attention(q, k, v, mask=mask[rows], bias=bias))
    weighted *= torch.sigmoid(module.gating_query(x))
    return module.output_projection(weighted)


class Transition(nn.Module):
    """``xfold/nn/primitives.py:20-37``: LN -> GLU(transition1.weight.T) -> transition2."""

    def __init__(self, c_x: int, num_intermediate_factor: int = 4) -> None:
        super().__init__()
        self.num_intermediate_factor = num_intermediate_factor
        self.c_in = c_x
        self.input_layer_norm = LayerNorm(c_x)
        self.transition1 = nn.Linear(c_x, num_intermediate_factor * c_x * 2, bias=False)
        self.transition2 = nn.Linear(num_intermediate_factor * c_x, c_x, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.input_layer_norm(x)
        return self.transition2(gated_linear_unit(x, self.transition1.weight.T))


class OuterProductMean(nn.Module):
    """``xfold/nn/primitives.py:40-72``: LN(msa) -> masked left/right projections ->
    out[i, j, f] = (sum_{c,e} (sum_s left[s,i,c] right[s,j,e]) output_w[c,e,f] + output_b[f])
    / (1e-3 + sum_s mask[s,i] mask[s,j]). The reference's einsum pair ('acb,ade->dceb',
    'dceb,cef->dbf', then permute(1, 0, 2)) is the same sum, indexed [j, ..., i] before the
    final transpose."""

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
        m = mask.unsqueeze(-1)                                    # [S, N, 1]
        x = self.layer_norm_input(msa)
        left = m * self.left_projection(x)                        # [S, N, c]
        right = m * self.right_projection(x)
        outer = torch.einsum("sic,sje->ijce", left, right)        # summed over sequences
        act = torch.einsum("ijce,cef->ijf", outer, self.output_w) + self.output_b
        norm = torch.einsum("si,sj->ij", mask, mask).unsqueeze(-1)
        return act / (self.epsilon + norm)


class MSAAttention(nn.Module):
    """``xfold/nn/attention.py:108-144``: attention weights from the pair alone,
    softmax(pair_logits(LN(pair)) + 1e9 (max_s msa_mask - 1)) over keys, shared by every
    MSA row; each row averages its own values v = v_projection(LN(msa)) per head, gated by
    sigmoid(gating_query(LN(msa))), then output_projection."""

    def __init__(self, c_msa: int = 64, c_pair: int = 128, num_head: int = 8) -> None:
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
        x = self.act_norm(msa)
        logits = self.pair_logits(self.pair_norm(pair)).permute(2, 0, 1)     # [H, q, k]
        logits = logits + 1e9 * (msa_mask.max(dim=0).values - 1.0)            # masked keys
        weights = torch.softmax(logits, dim=-1)
        rows, n = x.shape[0], x.shape[1]
        v = self.v_projection(x).reshape(rows, n, self.num_head, self.value_dim)
        avg = torch.einsum("hqk,skhc->sqhc", weights, v).reshape(rows, n, self.c_msa)
        avg = avg * torch.sigmoid(self.gating_query(x))
        return self.output_projection(avg)


class AdaptiveLayerNorm(nn.Module):
    """``xfold/nn/diffusion_transformer.py:27-64``.

    Conditioned: ``sigmoid(scale(LN_w(cond))) * LN_noaffine(x) + bias(LN_w(cond))``
    (:57-62); the x-norm has no affine (:40-41), the cond-norm has weight only (:42-43).
    Unconditioned: a plain affine LayerNorm (:48-49, :64).
    """

    def __init__(self, c_x: int, c_single_cond: int, use_single_cond: bool = False) -> None:
        super().__init__()
        self.c_x = c_x
        self.c_single_cond = c_single_cond
        self.use_single_cond = use_single_cond
        if use_single_cond:
            self.layer_norm = LayerNorm(c_x, elementwise_affine=False, bias=False)
            self.single_cond_layer_norm = LayerNorm(c_single_cond, bias=False)
            self.single_cond_scale = nn.Linear(c_single_cond, c_x, bias=True)
            self.single_cond_bias = nn.Linear(c_single_cond, c_x, bias=False)
        else:
            self.layer_norm = LayerNorm(c_x)

    def forward(self, x: torch.Tensor, single_cond: Optional[torch.Tensor] = None) -> torch.Tensor:
        assert (single_cond is None) == (not self.use_single_cond)
        if not self.use_single_cond:
            return self.layer_norm(x)
        x = self.layer_norm(x)
        cond = self.single_cond_layer_norm(single_cond)
        return torch.sigmoid(self.single_cond_scale(cond)) * x + self.single_cond_bias(cond)


class AdaLNZero(nn.Module):
    """``xfold/nn/diffusion_transformer.py:67-95``: transition2(x), gated by
    sigmoid(adaptive_zero_cond(cond)) when conditioned (:91-94)."""

    def __init__(self, c_in: int, c_out: int, c_single_cond: int, use_single_cond: bool = False):
        super().__init__()
        self.c_in = c_in
        self.c_out = c_out
        self.c_single_cond = c_single_cond
        self.use_single_cond = use_single_cond
        self.transition2 = nn.Linear(c_in, c_out, bias=False)
        if use_single_cond:
            self.adaptive_zero_cond = nn.Linear(c_single_cond, c_out, bias=True)

    def forward(self, x: torch.Tensor, single_cond: Optional[torch.Tensor] = None) -> torch.Tensor:
        assert (single_cond is None) == (not self.use_single_cond)
        out = self.transition2(x)
        if self.use_single_cond:
            out = torch.sigmoid(self.adaptive_zero_cond(single_cond)) * out
        return out


class DiffusionTransition(nn.Module):
    """``xfold/nn/diffusion_transformer.py:98-128``: AdaptiveLN -> GLU -> AdaLNZero."""

    def __init__(self, c_x: int, c_single_cond: int, num_intermediate_factor: int = 2,
                 use_single_cond: bool = False) -> None:
        super().__init__()
        self.c_x = c_x
        self.c_single_cond = c_single_cond
        self.num_intermediate_factor = num_intermediate_factor
        self.use_single_cond = use_single_cond
        self.adaptive_layernorm = AdaptiveLayerNorm(c_x, c_single_cond, use_single_cond)
        self.transition1 = nn.Linear(c_x, 2 * c_x * num_intermediate_factor, bias=False)
        self.adaptive_zero_init = AdaLNZero(num_intermediate_factor * c_x, c_x, c_single_cond,
                                            use_single_cond)

    def forward(self, x: torch.Tensor, single_cond: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = self.adaptive_layernorm(x, single_cond)
        hidden = gated_linear_unit(x, self.transition1.weight.T)
        return self.adaptive_zero_init(hidden, single_cond)


class SelfAttention(nn.Module):
    """``xfold/nn/diffusion_transformer.py:131-217`` (torch path :184-217).

    AdaptiveLN -> q (with bias), k, v -> 'n (h c) -> h n c' + batch dim -> attention with
    ``bias=pair_logits`` and a 1-D key mask -> gate with sigmoid(gating_query(x)) ->
    AdaLNZero. ``x`` is ``[N, c]`` (one diffusion sample); a leading sample dim is
    evaluated sample by sample, which is what the reference does (one call per sample).
    """

    def __init__(self, c_x: int = 768, c_single_cond: int = 384, num_head: int = 16,
                 use_single_cond: bool = False) -> None:
        super().__init__()
        self.c_x = c_x
        self.c_single_cond = c_single_cond
        self.num_head = num_head
        self.qkv_dim = c_x // num_head
        self.use_single_cond = use_single_cond
        self.adaptive_layernorm = AdaptiveLayerNorm(c_x, c_single_cond, use_single_cond)
        self.q_projection = nn.Linear(c_x, c_x, bias=True)
        self.k_projection = nn.Linear(c_x, c_x, bias=False)
        self.v_projection = nn.Linear(c_x, c_x, bias=False)
        self.gating_query = nn.Linear(c_x, c_x, bias=False)
        self.adaptive_zero_init = AdaLNZero(c_x, c_x, c_single_cond, use_single_cond)

    def forward(self, x: torch.Tensor, mask: torch.Tensor, pair_logits: Optional[torch.Tensor] = None,
                single_cond: Optional[torch.Tensor] = None, attention=None) -> torch.Tensor:
        if x.dim() == 3:
            return torch.stack([self.forward(sample, mask, pair_logits, single_cond, attention)
                                for sample in x])
        attention = attention or dot_product_attention
        assert (single_cond is None) == (not self.use_single_cond)
        x = self.adaptive_layernorm(x, single_cond)
        q = _heads_first(self.q_projection(x), self.num_head).unsqueeze(0)
        k = _heads_first(self.k_projection(x), self.num_head).unsqueeze(0)
        v = _heads_first(self.v_projection(x), self.num_head).unsqueeze(0)
        weighted = attention(q, k, v, mask=mask, bias=pair_logits).squeeze(0)
        weighted = _heads_last(weighted)
        weighted *= torch.sigmoid(self.gating_query(x))
        return self.adaptive_zero_init(weighted, single_cond)


class CrossAttention(nn.Module):
    """``xfold/nn/diffusion_transformer.py:275-350``: attention of atom-query subsets over
    atom-key subsets (x_q [..., Q, key_dim], x_k [..., K, key_dim], masks [..., Q] / [..., K]).

    q = q_projection(AdaLN_q(x_q, cond_q)) (with bias), k and v from AdaLN_k(x_k, cond_k);
    logits[h, q, k] = (q_scale q) . k + 1e9 [mask_q[q] == 0 and mask_k[k] == 0] (+ pair_logits)
    (:318-339): the 1e9 term is positive, so a masked query attends to the masked keys only
    and an unmasked query to every key. Softmax over keys, gate with
    sigmoid(gating_query(AdaLN_q(x_q))), AdaLNZero conditioned on cond_q (:341-350).
    """

    def __init__(self, key_dim: int = 128, value_dim: int = 128, c_single_cond: int = 128,
                 num_head: int = 4) -> None:
        super().__init__()
        self.key_dim = key_dim
        self.value_dim = value_dim
        self.c_single_cond = c_single_cond
        self.num_head = num_head
        self.key_dim_per_head = key_dim // num_head
        self.value_dim_per_head = value_dim // num_head
        self.q_scale = self.key_dim_per_head ** -0.5
        self.q_adaptive_layernorm = AdaptiveLayerNorm(key_dim, c_single_cond, use_single_cond=True)
        self.k_adaptive_layernorm = AdaptiveLayerNorm(key_dim, c_single_cond, use_single_cond=True)
        self.q_projection = nn.Linear(key_dim, key_dim, bias=True)
        self.k_projection = nn.Linear(key_dim, key_dim, bias=False)
        self.v_projection = nn.Linear(value_dim, value_dim, bias=False)
        self.gating_query = nn.Linear(key_dim, value_dim, bias=False)
        self.adaptive_zero_init = AdaLNZero(value_dim, value_dim, key_dim, use_single_cond=True)

    def forward(self, x_q, x_k, mask_q, mask_k, pair_logits=None, single_cond_q=None, single_cond_k=None):
        both_masked = ((mask_q == 0).unsqueeze(-1) & (mask_k == 0).unsqueeze(-2)).unsqueeze(-3)
        xq = self.q_adaptive_layernorm(x_q, single_cond_q)
        xk = self.k_adaptive_layernorm(x_k, single_cond_k)
        h = self.num_head
        q = self.q_projection(xq).unflatten(-1, (h, self.key_dim_per_head))
        k = self.k_projection(xk).unflatten(-1, (h, self.key_dim_per_head))
        logits = torch.einsum("...qhc,...khc->...hqk", q * self.q_scale, k) + 1e9 * both_masked
        if pair_logits is not None:
            logits = logits + pair_logits
        weights = torch.softmax(logits, dim=-1)
        v = self.v_projection(xk).unflatten(-1, (h, self.value_dim_per_head))
        avg = torch.einsum("...hqk,...khc->...qhc", weights, v).flatten(-2)
        avg = avg * torch.sigmoid(self.gating_query(xq))
        return self.adaptive_zero_init(avg, single_cond_q)


class PairformerBlock(nn.Module):
    """``xfold/nn/pairformer.py:26-114``.

    Five in-place residual updates of ``pair`` in order (:96-100), each op seeing the
    updated pair; then (with_single) pair logits = Linear(LN(pair)) permuted to [H, N, N]
    (:103-106), ``single += SelfAttention(single, seq_mask, pair_logits)`` (:108-110) and
    ``single += Transition(single)`` (:112).
    """

    def __init__(self, n_heads: int = 16, c_pair: int = 128, c_single: int = 384,
                 c_hidden_mul: int = 128, n_heads_pair: int = 4, num_intermediate_factor: int = 4,
                 with_single: bool = True) -> None:
        super().__init__()
        self.n_heads = n_heads
        self.with_single = with_single
        self.num_intermediate_factor = num_intermediate_factor
        self.triangle_multiplication_outgoing = TriangleMultiplication(c_pair, _outgoing=True)
        self.triangle_multiplication_incoming = TriangleMultiplication(c_pair, _outgoing=False)
        self.pair_attention1 = GridSelfAttention(c_pair, n_heads_pair, transpose=False)
        self.pair_attention2 = GridSelfAttention(c_pair, n_heads_pair, transpose=True)
        self.pair_transition = Transition(c_pair, num_intermediate_factor)
        self.c_single = c_single
        if with_single:
            self.single_pair_logits_norm = LayerNorm(c_pair)
            self.single_pair_logits_projection = nn.Linear(c_pair, n_heads, bias=False)
            self.single_attention_ = SelfAttention(c_single, num_head=n_heads, use_single_cond=False)
            self.single_transition = Transition(c_single)

    def forward(self, pair, pair_mask, single=None, seq_mask=None, attention=None):
        attn = attention
        pair += self.triangle_multiplication_outgoing(pair, mask=pair_mask)
        pair += self.triangle_multiplication_incoming(pair, mask=pair_mask)
        pair += self.pair_attention1(pair, mask=pair_mask, attention=attn)
        pair += self.pair_attention2(pair, mask=pair_mask, attention=attn)
        pair += self.pair_transition(pair)
        if not self.with_single:
            return pair
        logits = self.single_pair_logits_projection(self.single_pair_logits_norm(pair))
        logits = logits.permute(2, 0, 1)
        single += self.single_attention_(single, seq_mask, pair_logits=logits, attention=attn)
        single += self.single_transition(single)
        return pair, single


class EvoformerBlock(nn.Module):
    """``xfold/nn/pairformer.py:117-156``: pair += OuterProductMean(msa); msa +=
    MSAAttention(msa, pair); msa += Transition(msa); then the five pair updates of the
    Pairformer block (:149-154), each seeing the updated tensors."""

    def __init__(self, c_msa: int = 64, c_pair: int = 128, n_heads_pair: int = 4) -> None:
        super().__init__()
        self.outer_product_mean = OuterProductMean(c_msa=c_msa, num_output_channel=c_pair)
        self.msa_attention1 = MSAAttention(c_msa=c_msa, c_pair=c_pair)
        self.msa_transition = Transition(c_msa)
        self.triangle_multiplication_outgoing = TriangleMultiplication(c_pair, _outgoing=True)
        self.triangle_multiplication_incoming = TriangleMultiplication(c_pair, _outgoing=False)
        self.pair_attention1 = GridSelfAttention(c_pair, n_heads_pair, transpose=False)
        self.pair_attention2 = GridSelfAttention(c_pair, n_heads_pair, transpose=True)
        self.pair_transition = Transition(c_pair)

    def forward(self, msa, pair, msa_mask, pair_mask, attention=None):
        pair += self.outer_product_mean(msa, msa_mask)
        msa += self.msa_attention1(msa, msa_mask, pair)
        msa += self.msa_transition(msa)
        pair += self.triangle_multiplication_outgoing(pair, mask=pair_mask)
        pair += self.triangle_multiplication_incoming(pair, mask=pair_mask)
        pair += self.pair_attention1(pair, mask=pair_mask, attention=attention)
        pair += self.pair_attention2(pair, mask=pair_mask, attention=attention)
        pair += self.pair_transition(pair)
        return msa, pair


class DiffusionTransformer(nn.Module):
    """``xfold/nn/diffusion_transformer.py:220-272``.

    pair_act = LN(pair_cond) (:256-258); per super-block s the pair logits are
    ``Linear_s(pair_act)`` viewed 'n s (b h) -> b h n s' with h = num_head (:260-265), and
    block ``s*size + j`` uses logits[j] (:266-270). Every SelfAttention has 16 heads (the
    module's default, :244-245). The reference's InputCache only memoises these values.
    """

    def __init__(self, c_act: int = 768, c_single_cond: int = 384, c_pair_cond: int = 128,
                 num_head: int = 16, num_blocks: int = 24, super_block_size: int = 4) -> None:
        super().__init__()
        self.c_act = c_act
        self.c_single_cond = c_single_cond
        self.c_pair_cond = c_pair_cond
        self.num_head = num_head
        self.num_blocks = num_blocks
        self.super_block_size = super_block_size
        self.num_super_blocks = num_blocks // super_block_size
        self.pair_input_layer_norm = LayerNorm(c_pair_cond)
        self.pair_logits_projection = nn.ModuleList(
            [nn.Linear(c_pair_cond, super_block_size * num_head, bias=False)
             for _ in range(self.num_super_blocks)])
        # The pair logits are an autocast Linear's output, kept between the sampler's calls
        # (:255-265): bf16 under bf16 autocast. oracle.bf16_floor rounds the outputs of a
        # Linear whose weight carries this mark; the exact evaluation ignores it.
        for projection in self.pair_logits_projection:
            projection.weight._bf16_linear_output = True
        self.self_attention = nn.ModuleList(
            [SelfAttention(c_act, c_single_cond, use_single_cond=True) for _ in range(num_blocks)])
        self.transition_block = nn.ModuleList(
            [DiffusionTransition(c_act, c_single_cond, use_single_cond=True)
             for _ in range(num_blocks)])

    def super_block_logits(self, pair_act: torch.Tensor, s: int) -> torch.Tensor:
        projected = self.pair_logits_projection[s](pair_act)          # [n, s, (b h)]
        n, m, _ = projected.shape
        projected = projected.reshape(n, m, self.super_block_size, self.num_head)
        return projected.permute(2, 3, 0, 1)                          # [b, h, n, s]

    def forward(self, act, mask, single_cond, pair_cond, attention=None):
        pair_act = self.pair_input_layer_norm(pair_cond)
        for s in range(self.num_super_blocks):
            logits = self.super_block_logits(pair_act, s)
            for j in range(self.super_block_size):
                index = s * self.super_block_size + j
                act += self.self_attention[index](act, mask, logits[j], single_cond, attention=attention)
                act += self.transition_block[index](act, single_cond)
        return act


def rms(t: torch.Tensor) -> float:
    t = t.detach().to(torch.float64)
    return math.sqrt(float((t * t).mean())) if t.numel() else 0.0
