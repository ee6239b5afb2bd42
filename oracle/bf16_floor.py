"""The error floor of bf16 matrix arithmetic (test infrastructure only).

Each function re-evaluates a reference operator in float64 with ONLY the operands of its
matrix products rounded to bf16 (activations and weights entering a matmul, attention
probabilities and values), plus the two intermediates that the reference's own bf16
backends hold in bf16 between their GEMMs: the triangle-multiplication contraction
(``af3_kernels/src/csrc/triangle_multiplication.cpp:61-63``, a ``tiled_matmul`` result in
the compute dtype; ``torch.einsum`` under autocast) and the attention output P.V
(``af3_kernels/src/csrc/dot_product_attention.cpp:99-102``, a GEMM into the output dtype).
Accumulation is float64 and every other step exact. No implementation that feeds bf16
operands to matrix cores and keeps those two tensors in bf16 can be systematically more
accurate; the distance of this result from the exact (float64) operator is the floor
against which the HIP bf16 path is judged.

Follows the same reference lines as ``oracle.restatement``:
  triangle_multiplication   xfold/nn/triangle_multiplication.py:71-105
  grid_self_attention       xfold/nn/attention.py:61-105, xfold/fastnn/attention.py:45-66
  transition                xfold/nn/primitives.py:33-37
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import restatement as R


def _r(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float64)


def _lin(x, w):
    return _r(x) @ _r(w).T


def _ln(x, m):
    w = None if m.weight is None else m.weight.double()
    b = None if m.bias is None else m.bias.double()
    return F.layer_norm(x, (x.shape[-1],), w, b, m.eps)


def triangle_multiplication(m, pair, mask):
    x = _ln(pair.double(), m.left_norm_input)
    p = _lin(x, m.projection.weight).permute(2, 0, 1)
    if mask is not None:
        p = p * mask.double()[None]
    p = p * torch.sigmoid(_lin(x, m.gate.weight).permute(2, 0, 1))
    p = p.reshape(m.c_pair, 2, *p.shape[1:])
    out = _r(torch.einsum(m.equation, _r(p[:, 0]), _r(p[:, 1]))).permute(1, 2, 0)
    out = _lin(_ln(out, m.center_norm), m.output_projection.weight)
    return out * torch.sigmoid(_lin(x, m.gating_linear.weight))


def grid_self_attention(m, pair, mask):
    x = _ln(pair.double(), m.act_norm)
    bias = _lin(x, m.pair_bias_projection.weight).permute(2, 0, 1)
    if m.transpose:
        x = x.permute(1, 0, 2)
    q, k, v = (R._heads_first(_lin(x, getattr(m, n).weight), m.num_head)
               for n in ("q_projection", "k_projection", "v_projection"))
    logits = _r(q * q.shape[-1] ** -0.5) @ _r(k).transpose(-1, -2) + bias
    logits = logits.masked_fill(~mask.bool()[:, None, None, :], -1e9)
    o = R._heads_last(_r(_r(torch.softmax(logits, -1)) @ _r(v)))
    o = _lin(o * torch.sigmoid(_lin(x, m.gating_query.weight)), m.output_projection.weight)
    return o.permute(1, 0, 2) if m.transpose else o


def transition(m, x):
    x = _ln(x.double(), m.input_layer_norm)
    gate, value = _lin(x, m.transition1.weight).chunk(2, dim=-1)
    return _lin(F.silu(gate) * value, m.transition2.weight)


# ----------------------------------------------------------------------------------------
# The same floor for any composition of the restatement's modules
# ----------------------------------------------------------------------------------------

from torch.overrides import TorchFunctionMode  # noqa: E402

# Matrix products whose operands a bf16 matrix-core implementation rounds. For `linear`
# only the input and the weight are operands; the bias is added to the fp32 accumulator.
_PRODUCTS = {"linear", "matmul", "__matmul__", "__rmatmul__", "einsum", "bmm", "mm"}


def _round_operand(t):
    if isinstance(t, torch.Tensor) and t.is_floating_point():
        return t.to(torch.bfloat16).to(t.dtype)
    if isinstance(t, (list, tuple)):
        return type(t)(_round_operand(x) for x in t)
    return t


def _to_float64(t):
    if isinstance(t, torch.Tensor) and t.dtype == torch.float32:
        return t.to(torch.float64)
    if isinstance(t, (list, tuple)):
        return type(t)(_to_float64(x) for x in t)
    return t


def mark_residual(t: torch.Tensor) -> torch.Tensor:
    """Marks ``t`` as a bf16 residual stream for :class:`Bf16Operands`: every in-place
    update ``t += update`` under the mode is rounded to bf16, as an update of a bf16 pair,
    single or diffusion activation is (``xfold/nn/pairformer.py:96-112`` and
    ``xfold/nn/diffusion_transformer.py:266-270`` keep the caller's dtype). Returns ``t``."""
    t._bf16_residual = True
    return t


class Bf16Operands(TorchFunctionMode):
    """While active, every matrix product of the restatement (``nn.Linear``'s
    ``F.linear``, ``torch.matmul``/``@``, ``torch.einsum``, ``bmm``/``mm``) sees its
    operands rounded to bf16 and keeps its accumulation in the caller's dtype (fp32 or
    float64); the contraction (the restatement's only ``einsum``), the attention output
    (a product whose left operand is a softmax) and the output of a Linear whose weight is
    marked ``_bf16_linear_output`` (the DiffusionTransformer's pair logits, an autocast
    Linear output the reference keeps between calls) are rounded to bf16 as well; LayerNorm,
    softmax, sigmoid, the mask fill and the residual adds stay exact, except that an
    in-place add into a tensor marked by :func:`mark_residual` is rounded to bf16
    afterwards. Running ``oracle.restatement``'s modules under this mode
    gives the bf16 floor of any composition of them (a whole PairformerBlock, the 24-block
    DiffusionTransformer) in the same sense as the per-operator functions above, which it
    reproduces (tests/test_oracle.py)."""

    def __init__(self, float64: bool = False):
        super().__init__()
        self.float64 = float64

    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = getattr(func, "__name__", "")
        marked = name == "linear" and getattr(args[1] if len(args) > 1 else kwargs.get("weight"),
                                              "_bf16_linear_output", False)
        if self.float64 and not name.endswith("_"):
            # Every out-of-place op evaluates in float64 (fp32 parameters and inputs are
            # exact in it): the same floor with another accumulation precision, hence
            # another realization of its rounding pattern.
            args, kwargs = _to_float64(args), {k: _to_float64(v) for k, v in kwargs.items()}
        if name in ("add_", "__iadd__") and getattr(args[0], "_bf16_residual", False):
            out = func(*args, **kwargs)
            out.copy_(out.to(torch.bfloat16))
            return out
        if name == "softmax":
            out = func(*args, **kwargs)
            out._softmax_output = True
            return out
        if name not in _PRODUCTS:
            return func(*args, **kwargs)
        stored = name == "einsum" or getattr(args[0], "_softmax_output", False)
        if name == "linear":
            stored = stored or marked
            args = tuple(_round_operand(a) if i < 2 else a for i, a in enumerate(args))
            if "weight" in kwargs:
                kwargs = dict(kwargs, weight=_round_operand(kwargs["weight"]))
        elif name == "einsum":
            args = (args[0],) + tuple(_round_operand(a) for a in args[1:])
        else:
            args = tuple(_round_operand(a) for a in args)
        out = func(*args, **kwargs)
        return _round_operand(out) if stored else out
