"""The reference's native (cpp) backend restated for the CPU baseline (test infrastructure).

``oracle/cpp/af3_port.cpp`` restates af3_kernels' algorithms (``af3_kernels/src/csrc/*.cpp``)
as a PyTorch C++ extension: OpenMP over 128 x 128 output tiles, each tile's GEMM by ATen
(oneDNN) instead of LIBXSMM. This module builds and loads it and restates the Python side
of the reference's cpp path: ``linear_cpp`` (``xfold/fastnn/native.py:55-70``),
``dot_product_attention_cpp`` (``xfold/fastnn/attention.py:8-30``) and the modules' cpp
branches, composed into the Pairformer block and the diffusion transformer the way the
reference composes them with every switch on ``cpp``:

  TriangleMultiplication._forward_cpp      xfold/nn/triangle_multiplication.py:48-69
  GridSelfAttention._attention_cpp         xfold/nn/attention.py:49-59 (LayerNorm and the bias
                                           projection stay torch, :89-95)
  Transition                               xfold/nn/primitives.py:33-37 (GLU cpp, transition2 torch)
  SelfAttention._forward_cpp               xfold/nn/diffusion_transformer.py:170-182
  DiffusionTransition                      xfold/nn/diffusion_transformer.py:124-128 (GLU cpp)

It is timed by bench.py's ``cpu_baseline`` (the "cpp" leg) and checked against
``oracle.restatement`` by tests/test_cpp_port.py; nothing under xfold_cpu_amd/ uses it.
"""

from __future__ import annotations

import importlib.machinery
import importlib.util
from pathlib import Path

import torch

from . import restatement as R

SOURCE = Path(__file__).resolve().parent / "cpp" / "af3_port.cpp"
BUILD_DIR = Path(__file__).resolve().parent / "_cpp_build"
NAME = "af3_port"
_EXT = None


def build(verbose: bool = False):
    """Compiles the extension into oracle/_cpp_build/ (g++ -O3 -fopenmp, no -march, so the
    object runs on any x86-64 host)."""
    from torch.utils.cpp_extension import load
    BUILD_DIR.mkdir(exist_ok=True)
    return load(name=NAME, sources=[str(SOURCE)], build_directory=str(BUILD_DIR),
                extra_cflags=["-O3", "-fopenmp"], extra_ldflags=["-fopenmp"], verbose=verbose)


def load():
    """The built extension (no compilation: RuntimeError when it has not been built)."""
    global _EXT
    if _EXT is None:
        path = BUILD_DIR / f"{NAME}.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built (oracle.cpp_port.build())")
        loader = importlib.machinery.ExtensionFileLoader(NAME, str(path))
        spec = importlib.util.spec_from_file_location(NAME, str(path), loader=loader)
        module = importlib.util.module_from_spec(spec)
        loader.exec_module(module)
        _EXT = module
    return _EXT


def _dtype(*tensors):
    """``compute_dtype`` (xfold/fastnn/native.py:31-43): the CPU autocast dtype when enabled."""
    if torch.is_autocast_enabled("cpu"):
        return torch.get_autocast_dtype("cpu")
    return tensors[0].dtype


def _prep(t, dtype=None):
    if t is None:
        return None
    t = t.detach()
    return (t.to(dtype) if dtype is not None else t).contiguous()


def linear_cpp(x, layer):
    """``linear_cpp`` (xfold/fastnn/native.py:55-70): weight.T and bias in the compute dtype."""
    dtype = _dtype(x)
    with torch.amp.autocast("cpu", enabled=False):
        lead = x.shape[:-1]
        out = load().tiled_matmul(_prep(x, dtype).reshape(-1, x.shape[-1]), _prep(layer.weight.T, dtype),
                                  _prep(layer.bias, dtype))
        return out.reshape(*lead, out.shape[-1])


def gated_linear_unit_cpp(x, weight):
    """``gated_linear_unit`` with the cpp backend (xfold/fastnn/gated_linear_unit.py:110-122)."""
    dtype = _dtype(x)
    with torch.amp.autocast("cpu", enabled=False):
        lead = x.shape[:-1]
        out = load().gated_linear_unit(_prep(x, dtype).reshape(-1, x.shape[-1]), _prep(weight, dtype))
        return out.reshape(*lead, out.shape[-1])


def dot_product_attention_cpp(q, k, v, mask=None, bias=None):
    """xfold/fastnn/attention.py:8-30 and the extension's mask/bias broadcast
    (dot_product_attention.cpp:131-145): q scaled before the cast, bias fp32."""
    dtype = _dtype(q)
    with torch.amp.autocast("cpu", enabled=False):
        scaled = q.detach() * (q.size(-1) ** -0.5)
        b, h, nq, nk = q.size(0), q.size(1), q.size(2), k.size(2)
        m = None
        if mask is not None:
            m = mask.to(torch.bool)
            m = m.view(1, 1, 1, -1) if m.dim() == 1 else m[:, None, None, :] if m.dim() == 2 else m
            m = m.expand(b, h, nq, nk)
        bb = None if bias is None else bias.detach().to(torch.float32).expand(b, h, nq, nk)
        return load().dot_product_attention(_prep(scaled, dtype), _prep(k, dtype), _prep(v, dtype), m, bb)


def triangle_multiplication_cpp(m, pair, mask):
    """TriangleMultiplication._forward_cpp (xfold/nn/triangle_multiplication.py:48-69)."""
    dtype = _dtype(pair)
    with torch.amp.autocast("cpu", enabled=False):
        w = lambda layer: _prep(layer.weight.T, dtype)  # noqa: E731
        return load().triangle_multiplication(
            pair.detach().contiguous(), None if mask is None else mask.detach().to(dtype),
            m.equation == "cik,cjk->cij", m.left_norm_input.weight.detach(), m.left_norm_input.bias.detach(),
            w(m.projection), w(m.gate), m.center_norm.weight.detach(), m.center_norm.bias.detach(),
            w(m.output_projection), w(m.gating_linear), float(m.left_norm_input.eps),
            float(m.center_norm.eps), 128)


def grid_self_attention_cpp(m, pair, mask):
    """GridSelfAttention.forward with _attention_cpp (xfold/nn/attention.py:49-59, 80-105)."""
    normed = m.act_norm(pair)
    bias = m.pair_bias_projection(normed).permute(2, 0, 1)
    if m.transpose:
        normed = normed.permute(1, 0, 2)
    q, k, v = (R._heads_first(linear_cpp(normed, getattr(m, n)), m.num_head)
               for n in ("q_projection", "k_projection", "v_projection"))
    out = R._heads_last(dot_product_attention_cpp(q, k, v, mask=mask, bias=bias))
    out = out * torch.sigmoid(linear_cpp(normed, m.gating_query))
    out = linear_cpp(out, m.output_projection)
    return out.permute(1, 0, 2) if m.transpose else out


def grid_self_attention_rows_cpp(m, pair, mask, rows):
    """Batch rows ``rows`` of grid_self_attention_cpp (as oracle.restatement's
    grid_self_attention_rows: the bias from the whole normalised pair, q/k/v/gate from the
    selected rows), for a CPU sample at sizes where every row would take minutes."""
    normed = m.act_norm(pair)
    bias = m.pair_bias_projection(normed).permute(2, 0, 1)
    if m.transpose:
        normed = normed.permute(1, 0, 2)
    x = normed[rows]
    q, k, v = (R._heads_first(linear_cpp(x, getattr(m, n)), m.num_head)
               for n in ("q_projection", "k_projection", "v_projection"))
    out = R._heads_last(dot_product_attention_cpp(q, k, v, mask=mask[rows], bias=bias))
    out = out * torch.sigmoid(linear_cpp(x, m.gating_query))
    return linear_cpp(out, m.output_projection)


def transition_cpp(m, x):
    """Transition (xfold/nn/primitives.py:33-37): GLU cpp, transition2 a torch Linear."""
    return m.transition2(gated_linear_unit_cpp(m.input_layer_norm(x), m.transition1.weight.T))


def self_attention_cpp(m, x, mask, pair_logits=None, single_cond=None):
    """SelfAttention._forward_cpp (xfold/nn/diffusion_transformer.py:170-182)."""
    x = m.adaptive_layernorm(x, single_cond)
    q, k, v = (R._heads_first(linear_cpp(x, getattr(m, n)), m.num_head).unsqueeze(0)
               for n in ("q_projection", "k_projection", "v_projection"))
    out = R._heads_last(dot_product_attention_cpp(q, k, v, mask=mask, bias=pair_logits).squeeze(0))
    out = out * torch.sigmoid(linear_cpp(x, m.gating_query))
    return m.adaptive_zero_init(out, single_cond)


class PairformerBlockCpp:
    """PairformerBlock.forward (xfold/nn/pairformer.py:77-114) with every switch on cpp."""

    def __init__(self, block):
        self.b = block

    def __call__(self, pair, pair_mask, single=None, seq_mask=None, attention=None):
        b = self.b
        pair += triangle_multiplication_cpp(b.triangle_multiplication_outgoing, pair, pair_mask)
        pair += triangle_multiplication_cpp(b.triangle_multiplication_incoming, pair, pair_mask)
        pair += grid_self_attention_cpp(b.pair_attention1, pair, pair_mask)
        pair += grid_self_attention_cpp(b.pair_attention2, pair, pair_mask)
        pair += transition_cpp(b.pair_transition, pair)
        if not b.with_single:
            return pair
        logits = b.single_pair_logits_projection(b.single_pair_logits_norm(pair)).permute(2, 0, 1)
        single += self_attention_cpp(b.single_attention_, single, seq_mask, pair_logits=logits)
        single += transition_cpp(b.single_transition, single)
        return pair, single


class DiffusionTransformerCpp:
    """DiffusionTransformer.forward (xfold/nn/diffusion_transformer.py:250-272) with the
    attention and GLU switches on cpp."""

    def __init__(self, module):
        self.m = module

    def __call__(self, act, mask, single_cond, pair_cond):
        m = self.m
        pair_act = m.pair_input_layer_norm(pair_cond)
        for s in range(m.num_super_blocks):
            logits = m.super_block_logits(pair_act, s)
            for j in range(m.super_block_size):
                i = s * m.super_block_size + j
                act += self_attention_cpp(m.self_attention[i], act, mask, logits[j], single_cond)
                t = m.transition_block[i]
                x = t.adaptive_layernorm(act, single_cond)
                act += t.adaptive_zero_init(gated_linear_unit_cpp(x, t.transition1.weight.T), single_cond)
        return act
