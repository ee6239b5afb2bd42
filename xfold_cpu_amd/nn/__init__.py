"""HIP-backed modules with the reference's names, parameters and call signatures
(``xfold/nn/{triangle_multiplication,attention,primitives,pairformer,diffusion_transformer}.py``)."""

from .attention import GridSelfAttention, MSAAttention, grid_self_attention_hip, msa_attention_hip
from .diffusion_transformer import (AdaLNZero, AdaptiveLayerNorm, CrossAttention, DiffusionTransformer,
                                    DiffusionTransition, SelfAttention, cross_attention_hip,
                                    diffusion_transformer_hip, diffusion_transition_hip, self_attention_hip)
from .pairformer import EvoformerBlock, PairformerBlock, evoformer_block_hip, pairformer_block_hip
from .primitives import OuterProductMean, Transition, outer_product_mean_hip, transition_hip
from .triangle_multiplication import TriangleMultiplication, triangle_multiplication_hip

__all__ = [
    "AdaLNZero", "AdaptiveLayerNorm", "CrossAttention", "DiffusionTransformer", "DiffusionTransition", "EvoformerBlock",
    "GridSelfAttention", "MSAAttention", "OuterProductMean", "PairformerBlock", "SelfAttention",
    "Transition", "TriangleMultiplication",
    "cross_attention_hip", "diffusion_transformer_hip", "diffusion_transition_hip", "evoformer_block_hip", "grid_self_attention_hip",
    "msa_attention_hip", "outer_product_mean_hip", "pairformer_block_hip", "self_attention_hip",
    "transition_hip", "triangle_multiplication_hip",
]
