"""LayerNorm module with the reference's constructor and parameters
(``xfold/fastnn/layer_norm.py:14-53``), dispatching on ``config.layer_norm_implementation``
(``layer_norm.py:55-81``); this package implements the ``"hip"`` value."""

from __future__ import annotations

import numbers

import torch
import torch.nn as nn

from . import config as fastnn_config
from . import ops


class LayerNorm(nn.Module):
    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True,
                 bias: bool = True, device=None, dtype=None) -> None:
        factory = {"device": device, "dtype": dtype}
        super().__init__()
        if isinstance(normalized_shape, numbers.Integral):
            normalized_shape = (normalized_shape,)
        self.normalized_shape = tuple(normalized_shape)
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(self.normalized_shape, **factory))
            if bias:
                self.bias = nn.Parameter(torch.zeros(self.normalized_shape, **factory))
            else:
                self.register_parameter("bias", None)
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if fastnn_config.layer_norm_implementation != fastnn_config.HIP:
            raise ValueError("xfold_cpu_amd implements layer_norm_implementation='hip' only, "
                             f"got {fastnn_config.layer_norm_implementation!r}")
        if self.training:
            raise RuntimeError("The 'hip' LayerNorm supports eval inference only.")
        return ops.layer_norm(input, self.normalized_shape, self.weight, self.bias, self.eps, owner=self)

    def extra_repr(self) -> str:
        return f"{self.normalized_shape}, eps={self.eps}, elementwise_affine={self.elementwise_affine}"
