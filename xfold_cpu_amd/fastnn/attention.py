"""``dot_product_attention(q, k, v, mask=None, bias=None)`` with the reference's signature
and semantics (``xfold/fastnn/attention.py:45-98``): 3-D inputs gain a batch dim, q is
scaled by d^-0.5, bias is added, masked logits become -1e9, softmax over keys, @ v."""

from __future__ import annotations

from typing import Optional

import torch

from . import config as fastnn_config
from . import native_hip as nh
from . import ops


def dot_product_attention_hip(q, k, v, mask=None, bias=None):
    nh.check_gpu_inference(q, k, v, mask, bias)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or q.size(-1) == 0:
        raise ValueError("hip attention expects [B, H, Q/K, D] with positive head dims.")
    dtype = nh.compute_dtype(q, k, v)
    if mask is not None and mask.dim() not in (1, 2) and mask.dtype != torch.bool:
        raise ValueError("Attention masks of rank 0/3/4 must be boolean, as in the PyTorch path.")
    q, k, v = (t if t.dtype == dtype else ops.as_dtype(t, dtype) for t in (q, k, v))
    return ops.attention(q, k, v, mask, bias)


def dot_product_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          mask: Optional[torch.Tensor] = None,
                          bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    unbatched = q.dim() == 3
    if unbatched:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    if fastnn_config.dot_product_attention_implementation != fastnn_config.HIP:
        raise ValueError("Unknown dot_product_attention_implementation for xfold_cpu_amd: "
                         f"{fastnn_config.dot_product_attention_implementation!r} (only 'hip')")
    out = dot_product_attention_hip(q, k, v, mask, bias)
    return out.squeeze(0) if unbatched else out
