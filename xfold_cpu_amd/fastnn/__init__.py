"""HIP operators behind the reference's fastnn API (``xfold/fastnn/__init__.py:1-5``)."""

from .layer_norm import LayerNorm
from .attention import dot_product_attention
from .gated_linear_unit import gated_linear_unit

__all__ = ["LayerNorm", "dot_product_attention", "gated_linear_unit"]
