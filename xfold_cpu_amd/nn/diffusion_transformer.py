"""Diffusion-transformer modules with the reference's constructors, parameter names and
call signatures (``xfold/nn/diffusion_transformer.py:27-272``), running on the HIP backend:
AdaptiveLayerNorm, AdaLNZero, DiffusionTransition, SelfAttention (also the Pairformer's
single-track attention), DiffusionTransformer and the atom CrossAttention (:275-350).

The ``*_hip`` functions take any module carrying the reference's parameters. Activations
may carry a leading sample dim ([S, N, c]); conditioning tensors ([N, c_cond]) and pair
logits ([H, N, N]) are shared by all samples, which is what the reference computes one
sample at a time.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn as nn

from ..fastnn import LayerNorm
from ..fastnn import config as fastnn_config
from ..fastnn import native_hip as nh
from ..fastnn import ops
from .cache import InputCache


def _adaptive_layer_norm(aln: nn.Module, x: torch.Tensor, single_cond: Optional[torch.Tensor],
                         dtype: torch.dtype, out_dtype: Optional[torch.dtype] = None,
                         cond: Optional[tuple] = None) -> torch.Tensor:
    """``AdaptiveLayerNorm.forward`` (``diffusion_transformer.py:51-64``); Linears in
    ``dtype``, result in ``out_dtype`` (default ``dtype``). ``cond`` = (scale, shift) already
    computed from single_cond (see :func:`_block_conditioning`)."""
    if (single_cond is None) != (not aln.use_single_cond):
        raise ValueError("single_cond must be given exactly when use_single_cond is set")
    out_dtype = out_dtype or dtype
    if cond is not None:
        return ops.adaptive_layer_norm(x, cond[0], cond[1], aln.layer_norm.eps, out_dtype=out_dtype)
    if not aln.use_single_cond:
        ln = aln.layer_norm
        return ops.layer_norm(x, ln.normalized_shape, ln.weight, ln.bias, ln.eps, out_dtype=out_dtype,
                              owner=ln)
    cln = aln.single_cond_layer_norm
    cond = ops.layer_norm(single_cond, cln.normalized_shape, cln.weight, cln.bias, cln.eps,
                          out_dtype=dtype, owner=cln)
    # scale and shift stay fp32 (one rounding fewer before the sigmoid and the add).
    scale = ops.linear(cond, nh.linear_weight(aln, "single_cond_scale", dtype),
                       aln.single_cond_scale.bias, dtype, out_dtype=torch.float32)
    shift = ops.linear(cond, nh.linear_weight(aln, "single_cond_bias", dtype), None, dtype,
                       out_dtype=torch.float32)
    return ops.adaptive_layer_norm(x, scale, shift, aln.layer_norm.eps, out_dtype=out_dtype)


def _ada_ln_zero(zero: nn.Module, hidden: torch.Tensor, single_cond: Optional[torch.Tensor],
                 dtype: torch.dtype, accumulate_into: Optional[torch.Tensor],
                 cond: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``AdaLNZero.forward`` (``diffusion_transformer.py:85-95``), optionally added in place;
    ``cond`` = adaptive_zero_cond(single_cond) already computed, in the output dtype."""
    w = nh.linear_weight(zero, "transition2", dtype)
    out = accumulate_into
    out_dtype = out.dtype if out is not None else dtype
    acc = out is not None
    if zero.use_single_cond:
        if cond is None:
            cond = ops.linear(single_cond, nh.linear_weight(zero, "adaptive_zero_cond", dtype),
                              zero.adaptive_zero_cond.bias, dtype, out_dtype=out_dtype)
        epi = nh.EPI_MUL_SIGMOID_AUX_ACCUMULATE if acc else nh.EPI_MUL_SIGMOID_AUX
        return ops.linear(hidden, w, None, dtype, out=out, out_dtype=out_dtype, epilogue=epi,
                          aux=cond, aux_rows=cond.numel() // cond.shape[-1])
    epi = nh.EPI_ACCUMULATE if acc else nh.EPI_STORE
    return ops.linear(hidden, w, None, dtype, out=out, out_dtype=out_dtype, epilogue=epi)


def _check_accumulate(out, x):
    if out is not None and (not out.is_contiguous() or out.shape != x.shape):
        raise ValueError("accumulate_into must be a contiguous tensor shaped like x")


def diffusion_transition_hip(module: nn.Module, x: torch.Tensor, single_cond=None,
                             accumulate_into: Optional[torch.Tensor] = None, *,
                             _cond: Optional[tuple] = None) -> torch.Tensor:
    """``DiffusionTransition.forward`` (``diffusion_transformer.py:124-128``). ``_cond`` =
    (scale, shift, zero_cond) precomputed by :func:`_block_conditioning`."""
    nh.check_gpu_inference(x, single_cond)
    nh.check_module(module)
    dtype = nh.compute_dtype(x, module.transition1.weight)
    _check_accumulate(accumulate_into, x)
    xn = _adaptive_layer_norm(module.adaptive_layernorm, x, single_cond, dtype,
                              cond=None if _cond is None else _cond[:2])
    f = module.transition1.weight.shape[0] // 2
    hidden = ops.gated_linear_unit(xn, nh.linear_weight(module, "transition1", dtype, "glu"), f, dtype)
    return _ada_ln_zero(module.adaptive_zero_init, hidden, single_cond, dtype, accumulate_into,
                        cond=None if _cond is None else _cond[2])


_QKV = ("q_projection", "k_projection", "v_projection")


def _projection_bias(module: nn.Module, c: int, parts: int, device: torch.device) -> Optional[torch.Tensor]:
    """fp32 bias of the stacked [q | k | v (| gate)] projection: q_projection's bias, zeros
    for the rest (k, v and the gate have none), cached while the bias is unchanged."""
    q_bias = module.q_projection.bias
    if q_bias is None:
        return None
    cached = module.__dict__.get(f"_hip_proj_bias{parts}")
    key = (q_bias.data_ptr(), q_bias._version) if not q_bias.is_inference() else None
    if cached is None or key is None or cached[0] != key:
        full = torch.zeros(parts * c, dtype=torch.float32, device=device)
        full[:c] = q_bias.detach().to(torch.float32)
        cached = (key, full)
        if key is not None:
            module.__dict__[f"_hip_proj_bias{parts}"] = cached
    return cached[1]


_LOG2E = 1.4426950408889634


def self_attention_hip(module: nn.Module, x: torch.Tensor, mask: Optional[torch.Tensor],
                       pair_logits: Optional[torch.Tensor] = None,
                       single_cond: Optional[torch.Tensor] = None,
                       accumulate_into: Optional[torch.Tensor] = None, *,
                       _cond: Optional[tuple] = None,
                       _operands: Optional[ops.AttentionOperands] = None) -> torch.Tensor:
    """``SelfAttention.forward`` (``diffusion_transformer.py:184-217``) for x [N, c] or
    [S, N, c]; pair_logits [H, N, N] is the attention bias, mask [N] the key mask.
    ``_cond`` = (scale, shift, zero_cond) precomputed by :func:`_block_conditioning`.

    With bf16, a packed bias and head dims the pipelined kernel takes, the q/k/v and gating
    projections are one GEMM writing the attention kernel's layouts, and the gate is applied
    at the attention's store. ``_operands`` (an :class:`ops.AttentionOperands` of this shape,
    its mask words already set) lets a caller reuse one set of buffers over many blocks."""
    logits_t = pair_logits.tensor if isinstance(pair_logits, ops.PackedBias) else pair_logits
    nh.check_gpu_inference(x, mask, logits_t, single_cond)
    nh.check_module(module)
    dtype = nh.compute_dtype(x, *(getattr(module, n).weight for n in _QKV + ("gating_query",)))
    _check_accumulate(accumulate_into, x)
    if x.dim() not in (2, 3):
        raise ValueError("SelfAttention expects x [N, c] or [S, N, c]")
    samples = 1 if x.dim() == 2 else x.shape[0]
    n, c = x.shape[-2], x.shape[-1]
    heads = module.num_head
    d = c // heads
    xn = _adaptive_layer_norm(module.adaptive_layernorm, x, single_cond, dtype,
                              cond=None if _cond is None else _cond[:2])
    if dtype == torch.bfloat16 and isinstance(pair_logits, ops.PackedBias) and c % 32 == 0 and \
            ops.AttentionOperands.supported(n, heads, d) and \
            (mask is None or tuple(mask.shape) in ((n,), (samples, n))):
        operands = _operands
        if operands is None or not operands.matches(samples, n, heads, d, x.device):
            operands = ops.shared_attention_operands(samples, n, heads, d, x.device)
        operands.set_mask(mask)
        w_all = nh.fused_linear_weight(module, _QKV + ("gating_query",), dtype)
        ops.attention_project(xn, w_all, _projection_bias(module, c, 4, x.device), operands, d ** -0.5 * _LOG2E)
        o = ops.attention_on_operands(operands, pair_logits, torch.empty((samples, n, c), dtype=dtype, device=x.device))
        return _ada_ln_zero(module.adaptive_zero_init, o.reshape(x.shape), single_cond, dtype, accumulate_into,
                            cond=None if _cond is None else _cond[2])
    w_qkv = nh.fused_linear_weight(module, _QKV, dtype)
    bias_qkv = _projection_bias(module, c, 3, x.device)
    qkv = ops.linear(xn, w_qkv, bias_qkv, dtype)                     # [.., N, 3c]
    qkv = qkv.reshape(samples, n, 3 * c)
    row = 3 * c
    views = [torch.as_strided(qkv, (samples, heads, n, d), (n * row, d, row, 1), i * c)
             for i in range(3)]
    o = torch.empty((samples, n, c), dtype=dtype, device=x.device)
    o_view = torch.as_strided(o, (samples, heads, n, d), (n * c, d, c, 1), 0)
    bias = None
    if isinstance(pair_logits, ops.PackedBias):
        bias = pair_logits
    elif pair_logits is not None:
        bias = pair_logits if pair_logits.dim() == 4 else pair_logits.unsqueeze(0)
    ops.attention(views[0], views[1], views[2], mask, bias, out=o_view)
    ops.linear(xn.reshape(samples, n, c), nh.linear_weight(module, "gating_query", dtype), None, dtype,
               out=o, epilogue=nh.EPI_SIGMOID_MUL_AUX, aux=o)
    o = o.reshape(x.shape)
    return _ada_ln_zero(module.adaptive_zero_init, o, single_cond, dtype, accumulate_into,
                        cond=None if _cond is None else _cond[2])


def _conditioning_weights(module: nn.Module, alns, zeros, dtype: torch.dtype):
    """Stacked conditioning weights of every block (a cached one-time weight preparation):
    ([2A, c, c_s] scale/shift weights with the single_cond LayerNorm's weight folded into
    their input columns, [2A, c] fp32 biases, [Z, c, c_s] adaptive_zero_cond weights, [Z, c]
    biases). LayerNorm(s) = s_hat * g + b, so Linear(LayerNorm(s)) = s_hat (W g)^T + (W b + bias)."""
    srcs = []
    for a in alns:
        cln = a.single_cond_layer_norm
        srcs += [t for t in (cln.weight, cln.bias, a.single_cond_scale.weight, a.single_cond_scale.bias,
                             a.single_cond_bias.weight, a.single_cond_bias.bias) if t is not None]
    for z in zeros:
        srcs += [t for t in (z.adaptive_zero_cond.weight, z.adaptive_zero_cond.bias) if t is not None]

    def build(*_):
        with torch.no_grad():
            ws, bs = [], []
            for a in alns:
                cln = a.single_cond_layer_norm
                for lin in (a.single_cond_scale, a.single_cond_bias):
                    w = lin.weight.detach().float()
                    b = (lin.bias.detach().float() if lin.bias is not None
                         else torch.zeros(w.shape[0], dtype=torch.float32, device=w.device))
                    if cln.bias is not None:
                        b = b + w @ cln.bias.detach().float()
                    ws.append(w * cln.weight.detach().float() if cln.weight is not None else w)
                    bs.append(b)
            zw = [z.adaptive_zero_cond.weight.detach().float() for z in zeros]
            zb = [z.adaptive_zero_cond.bias.detach().float() if z.adaptive_zero_cond.bias is not None
                  else torch.zeros(w.shape[0], dtype=torch.float32, device=w.device)
                  for z, w in zip(zeros, zw)]
            return (torch.stack(ws).to(dtype).contiguous(), torch.stack(bs).contiguous(),
                    torch.stack(zw).to(dtype).contiguous(), torch.stack(zb).contiguous())

    return nh.derived_weight(module, f"conditioning:{dtype}", srcs, build)


def _block_conditioning(module: nn.Module, single_cond: torch.Tensor, dtype: torch.dtype,
                        zero_dtype: torch.dtype):
    """Every block's conditioning linears (``AdaptiveLayerNorm`` scale/shift,
    ``diffusion_transformer.py:59-62``; ``AdaLNZero`` cond, ``:93``) computed up front: they
    read only single_cond, which is the same for all blocks of one call. Two batched launches
    (one over the normalised single_cond, one over single_cond itself) replace the 6 small
    GEMMs of every block. Returns [(attention (scale, shift, zero), transition (...))] per
    block, or None when some block has no single_cond conditioning (the per-block path)."""
    n_blocks = len(module.self_attention)
    att = [module.self_attention[i] for i in range(n_blocks)]
    tr = [module.transition_block[i] for i in range(n_blocks)]
    alns = [b.adaptive_layernorm for b in att] + [b.adaptive_layernorm for b in tr]
    zeros = [b.adaptive_zero_init for b in att] + [b.adaptive_zero_init for b in tr]
    if single_cond is None or not all(a.use_single_cond for a in alns) or \
            not all(z.use_single_cond for z in zeros):
        return None
    eps = {a.single_cond_layer_norm.eps for a in alns}
    shapes = {tuple(a.single_cond_layer_norm.normalized_shape) for a in alns}
    if len(eps) != 1 or len(shapes) != 1:
        return None
    w_ss, b_ss, w_z, b_z = _conditioning_weights(module, alns, zeros, dtype)
    s_hat = ops.layer_norm(single_cond, shapes.pop(), None, None, eps.pop(), out_dtype=dtype)
    ss = ops.linear_batched(s_hat.reshape(-1, s_hat.shape[-1]), w_ss, b_ss, dtype)
    zz = ops.linear_batched(single_cond.reshape(-1, single_cond.shape[-1]), w_z, b_z, dtype,
                            out_dtype=zero_dtype)
    lead = single_cond.shape[:-1]
    view = lambda t: t.reshape(*lead, t.shape[-1])
    return [((view(ss[2 * i]), view(ss[2 * i + 1]), view(zz[i])),
             (view(ss[2 * (n_blocks + i)]), view(ss[2 * (n_blocks + i) + 1]), view(zz[n_blocks + i])))
            for i in range(n_blocks)]


def _cached(module: nn.Module, name: str, dependencies, factory, modules):
    """``module._input_cache.get`` (``xfold/nn/diffusion_transformer.py:255-265``) when the
    module carries an input cache (this package's or the reference's InputCache, which share
    the interface), else ``factory()``."""
    cache = getattr(module, "_input_cache", None)
    if cache is None:
        return factory()
    return cache.get(name, dependencies, module, factory, modules=modules)


def _block_operands(module: nn.Module, act: torch.Tensor, mask: Optional[torch.Tensor]):
    """The attention-operand buffers (and mask words) every block of a forward uses, or None
    when the blocks' attention takes the general path."""
    samples = 1 if act.dim() == 2 else act.shape[0]
    n, c, heads = act.shape[-2], act.shape[-1], module.num_head
    if c % heads or not ops.AttentionOperands.supported(n, heads, c // heads):
        return None
    if mask is not None and tuple(mask.shape) not in ((n,), (samples, n)):
        return None
    operands = ops.shared_attention_operands(samples, n, heads, c // heads, act.device)
    operands.set_mask(mask)
    return operands


def diffusion_transformer_hip(module: nn.Module, act: torch.Tensor, mask: torch.Tensor,
                              single_cond: torch.Tensor, pair_cond: torch.Tensor) -> torch.Tensor:
    """``DiffusionTransformer.forward`` (``diffusion_transformer.py:250-272``), updating
    ``act`` ([N, c] or [S, N, c], contiguous) in place and returning it.

    Inside an input-cache scope (``xfold_cpu_amd.nn.cache``, the reference's ``InputCache``
    rules) the packed pair logits of every super-block are kept across calls with the same
    ``pair_cond`` and weights, as the reference keeps its pair logits (``:255-265``), when
    they fit the scope's byte budget."""
    nh.check_gpu_inference(act, mask, single_cond, pair_cond)
    if not act.is_contiguous():
        raise ValueError("DiffusionTransformer (hip) updates act in place; pass a contiguous tensor")
    dtype = nh.compute_dtype(act, module.pair_logits_projection[0].weight)
    ln = module.pair_input_layer_norm
    heads, size = module.num_head, module.super_block_size
    # Not an input-cache entry: its key would cover ~400 parameters, whose checks cost more
    # host time than the two batched GEMMs they would save.
    conds = _block_conditioning(module, single_cond, dtype, act.dtype)
    n_blocks = module.num_super_blocks * size
    # A packed bias (either path below) feeds the pipelined attention kernel, which takes
    # bf16, head dims <= 64 and at most attention_max_keys() keys.
    packed_bias = dtype == torch.bfloat16 and act.shape[-1] // heads <= 64 and \
        pair_cond.shape[0] <= nh.attention_max_keys()
    if packed_bias and pair_cond.shape[-1] == 128 and n_blocks * heads <= 384 and \
            tuple(ln.normalized_shape) == (128,):
        # Every super-block's pair logits in one pass over pair_cond, straight into the
        # attention kernel's bias layout; block b reads heads b*H .. b*H + H - 1.
        projs = [module.pair_logits_projection[s].weight for s in range(module.num_super_blocks)]
        w_all = nh.derived_weight(module, f"pair_logits:{dtype}", projs,
                                  lambda *ws: torch.cat([w.detach() for w in ws], dim=0).to(dtype).contiguous())
        # bf16 logits, the dtype of the reference's autocast Linear output (half the bytes of
        # fp32: at N=768 all 24 blocks' logits take 453 MB and fit the input cache's budget).
        packed = _cached(module, "pair_logits_packed", (pair_cond, heads),
                         lambda: ops.pair_attention_bias(pair_cond, ln.weight, ln.bias, ln.eps, w_all, owner=ln,
                                                         out_dtype=torch.bfloat16),
                         modules=(ln, module.pair_logits_projection))
        operands = _block_operands(module, act, mask)
        for index in range(n_blocks):
            att_cond, tr_cond = (None, None) if conds is None else conds[index]
            bias = ops.PackedBias(packed[index * heads:(index + 1) * heads])
            self_attention_hip(module.self_attention[index], act, mask, bias, single_cond,
                               accumulate_into=act, _cond=att_cond, _operands=operands)
            diffusion_transition_hip(module.transition_block[index], act, single_cond,
                                     accumulate_into=act, _cond=tr_cond)
        return act
    pair_act = ops.layer_norm(pair_cond, ln.normalized_shape, ln.weight, ln.bias, ln.eps,
                              out_dtype=dtype, owner=ln)
    operands = _block_operands(module, act, mask) if packed_bias else None
    for s in range(module.num_super_blocks):
        weight = nh.linear_weight(module.pair_logits_projection, str(s), dtype)
        logits = ops.linear(pair_act, weight, None, dtype)               # [N, N, size*heads]
        # 'n s (b h) -> b h n s': block j, head h reads column j*heads + h. On the pipelined
        # attention path (bf16, head dim <= 64) the super-block's biases are converted once.
        n_tok = logits.shape[0]
        if packed_bias:
            packed = ops.attention_bias_pack(logits.view(n_tok, n_tok, size, heads).permute(2, 3, 0, 1))
        for j in range(size):
            if packed_bias:
                bias = ops.PackedBias(packed[j])
            else:
                bias = logits[..., j * heads:(j + 1) * heads].permute(2, 0, 1)
            index = s * size + j
            att_cond, tr_cond = (None, None) if conds is None else conds[index]
            self_attention_hip(module.self_attention[index], act, mask, bias, single_cond,
                               accumulate_into=act, _cond=att_cond, _operands=operands)
            diffusion_transition_hip(module.transition_block[index], act, single_cond,
                                     accumulate_into=act, _cond=tr_cond)
    return act


class AdaptiveLayerNorm(nn.Module):
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

    def forward(self, x, single_cond=None):
        _require(fastnn_config.layer_norm_implementation, "layer_norm_implementation")
        nh.check_gpu_inference(x, single_cond)
        dtype = nh.compute_dtype(x)
        # Under CUDA autocast the reference's LayerNorm output is fp32 and so is the
        # conditioned sum (fp32 * bf16 + bf16); outside autocast it is x's dtype.
        out_dtype = torch.float32 if torch.is_autocast_enabled("cuda") else x.dtype
        return _adaptive_layer_norm(self, x, single_cond, dtype, out_dtype)


class AdaLNZero(nn.Module):
    def __init__(self, c_in: int, c_out: int, c_single_cond: int, use_single_cond: bool = False):
        super().__init__()
        self.c_in = c_in
        self.c_out = c_out
        self.c_single_cond = c_single_cond
        self.use_single_cond = use_single_cond
        self.transition2 = nn.Linear(c_in, c_out, bias=False)
        if use_single_cond:
            self.adaptive_zero_cond = nn.Linear(c_single_cond, c_out, bias=True)

    def forward(self, x, single_cond=None):
        dtype = nh.compute_dtype(x, self.transition2.weight)
        return _ada_ln_zero(self, x, single_cond, dtype, None)


def _require(flag_value: str, what: str):
    if flag_value != fastnn_config.HIP:
        raise ValueError(f"Unknown {what} for xfold_cpu_amd: {flag_value!r} (only 'hip')")


class DiffusionTransition(nn.Module):
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

    def forward(self, x, single_cond=None):
        _require(fastnn_config.gated_linear_unit_implementation, "gated_linear_unit_implementation")
        return diffusion_transition_hip(self, x, single_cond)


class SelfAttention(nn.Module):
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

    def forward(self, x, mask, pair_logits=None, single_cond=None):
        _require(fastnn_config.dot_product_attention_implementation, "dot_product_attention_implementation")
        return self_attention_hip(self, x, mask, pair_logits, single_cond)


def cross_attention_hip(module: nn.Module, x_q: torch.Tensor, x_k: torch.Tensor, mask_q: torch.Tensor,
                        mask_k: torch.Tensor, pair_logits: Optional[torch.Tensor] = None,
                        single_cond_q: Optional[torch.Tensor] = None, single_cond_k: Optional[torch.Tensor] = None,
                        accumulate_into: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``CrossAttention.forward`` (``diffusion_transformer.py:304-350``) for x_q [..., Q, c],
    x_k [..., K, c] with masks [..., Q] / [..., K] and pair_logits broadcastable to
    [..., H, Q, K]: the q/k adaptive LayerNorms, the q and fused k|v projections, one
    attention over all subsets whose fp32 bias (pair logits + the reference's positive 1e9
    on pairs of a masked query and a masked key) comes from xfh_cross_attention_bias, the
    sigmoid gate as the gating Linear's epilogue and the conditioned AdaLNZero."""
    if mask_q.dim() != x_q.dim() - 1 or mask_k.dim() != x_k.dim() - 1:
        raise ValueError(f"CrossAttention: masks must drop the channel dim of x ({tuple(mask_q.shape)}, "
                         f"{tuple(x_q.shape)}; {tuple(mask_k.shape)}, {tuple(x_k.shape)})")
    nh.check_gpu_inference(x_q, x_k, mask_q, mask_k, pair_logits, single_cond_q, single_cond_k)
    nh.check_module(module)
    names = ("q_projection", "k_projection", "v_projection", "gating_query")
    dtype = nh.compute_dtype(x_q, *(getattr(module, n).weight for n in names))
    lead, nq, nk = tuple(x_q.shape[:-2]), x_q.shape[-2], x_k.shape[-2]
    if tuple(x_k.shape[:-2]) != lead:
        raise ValueError("CrossAttention: x_q and x_k must share their leading (subset) dims")
    batch = 1
    for d in lead:
        batch *= d
    h, dk, dv = module.num_head, module.key_dim_per_head, module.value_dim_per_head
    kd, vd = module.key_dim, module.value_dim
    if accumulate_into is not None and (not accumulate_into.is_contiguous() or
                                        tuple(accumulate_into.shape) != lead + (nq, vd)):
        raise ValueError("accumulate_into must be a contiguous [..., Q, value_dim] tensor")
    xq = _adaptive_layer_norm(module.q_adaptive_layernorm, x_q, single_cond_q, dtype)
    xk = _adaptive_layer_norm(module.k_adaptive_layernorm, x_k, single_cond_k, dtype)
    q = ops.linear(xq, nh.linear_weight(module, "q_projection", dtype), module.q_projection.bias, dtype)
    kv = ops.linear(xk, nh.fused_linear_weight(module, ("k_projection", "v_projection"), dtype), None, dtype)
    q4 = torch.as_strided(q, (batch, h, nq, dk), (nq * kd, dk, kd, 1))
    k4 = torch.as_strided(kv, (batch, h, nk, dk), (nk * (kd + vd), dk, kd + vd, 1))
    v4 = torch.as_strided(kv, (batch, h, nk, dv), (nk * (kd + vd), dv, kd + vd, 1), kd)
    mq, mq_code = nh.mask_arg(mask_q, lead + (nq,))
    mk, mk_code = nh.mask_arg(mask_k, lead + (nk,))
    bias = torch.empty((batch, h, nq, nk), dtype=torch.float32, device=x_q.device)
    pl, pl_code, strides = None, nh.F32, None
    if pair_logits is not None:
        if pair_logits.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("CrossAttention: pair_logits must be fp32 or bf16")
        pl = pair_logits.expand(*lead, h, nq, nk).reshape(batch, h, nq, nk)
        pl_code = nh.dtype_code(pl.dtype)
        strides = (ctypes.c_int64 * 4)(*pl.stride())
    nh.call("xfh_cross_attention_bias", nh.ptr(pl), pl_code, strides, nh.ptr(mq), mq_code, nh.ptr(mk), mk_code,
            batch, h, nq, nk, nh.ptr(bias), nh.stream_of(x_q.device))
    o = torch.empty(lead + (nq, vd), dtype=dtype, device=x_q.device)
    o_view = torch.as_strided(o, (batch, h, nq, dv), (nq * vd, dv, vd, 1))
    ops.attention(q4, k4, v4, None, bias, out=o_view, scale=module.q_scale)
    ops.linear(xq, nh.linear_weight(module, "gating_query", dtype), None, dtype, out=o,
               epilogue=nh.EPI_SIGMOID_MUL_AUX, aux=o)
    return _ada_ln_zero(module.adaptive_zero_init, o, single_cond_q, dtype, accumulate_into)


class CrossAttention(nn.Module):
    def __init__(self, key_dim: int = 128, value_dim: int = 128, c_single_cond: int = 128,
                 num_head: int = 4) -> None:
        super().__init__()
        self.key_dim = key_dim
        self.value_dim = value_dim
        self.c_single_cond = c_single_cond
        self.num_head = num_head
        self.key_dim_per_head = key_dim // num_head
        self.value_dim_per_head = value_dim // num_head
        self.q_scale = self.key_dim_per_head ** (-0.5)
        self.q_adaptive_layernorm = AdaptiveLayerNorm(key_dim, c_single_cond, use_single_cond=True)
        self.k_adaptive_layernorm = AdaptiveLayerNorm(key_dim, c_single_cond, use_single_cond=True)
        self.q_projection = nn.Linear(key_dim, key_dim, bias=True)
        self.k_projection = nn.Linear(key_dim, key_dim, bias=False)
        self.v_projection = nn.Linear(value_dim, value_dim, bias=False)
        self.gating_query = nn.Linear(key_dim, value_dim, bias=False)
        self.adaptive_zero_init = AdaLNZero(value_dim, value_dim, key_dim, use_single_cond=True)

    def forward(self, x_q, x_k, mask_q, mask_k, pair_logits=None, single_cond_q=None, single_cond_k=None):
        _require(fastnn_config.dot_product_attention_implementation, "dot_product_attention_implementation")
        return cross_attention_hip(self, x_q, x_k, mask_q, mask_k, pair_logits, single_cond_q, single_cond_k)


class DiffusionTransformer(nn.Module):
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
        self.self_attention = nn.ModuleList(
            [SelfAttention(c_act, c_single_cond, use_single_cond=True) for _ in range(num_blocks)])
        self.transition_block = nn.ModuleList(
            [DiffusionTransition(c_act, c_single_cond, use_single_cond=True) for _ in range(num_blocks)])
        self._input_cache = InputCache()

    def forward(self, act, mask, single_cond, pair_cond):
        _require(fastnn_config.dot_product_attention_implementation, "dot_product_attention_implementation")
        _require(fastnn_config.gated_linear_unit_implementation, "gated_linear_unit_implementation")
        _require(fastnn_config.layer_norm_implementation, "layer_norm_implementation")
        return diffusion_transformer_hip(self, act, mask, single_cond, pair_cond)
