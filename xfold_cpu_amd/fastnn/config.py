"""Backend selection, mirroring ``xfold/fastnn/config.py:1-16`` of the reference.

The reference reads these module globals at call time in every operator and module
(``xfold/nn/triangle_multiplication.py:41-46``, ``xfold/nn/attention.py:45,90``,
``xfold/nn/diffusion_transformer.py:166``, ``xfold/fastnn/*.py``). This package adds the
value ``"hip"`` and implements only that value: any other value raises ``ValueError``
from the operator that reads it (the reference's own ``torch``/``cpp``/``triton`` code
paths live in the reference package; there is no silent fallback).
"""

# options in the reference: ["torch", "triton", "ipex"]; this package: ["hip"]
layer_norm_implementation = "hip"

# options in the reference: ["torch", "triton", "cpp"]; this package: ["hip"]
dot_product_attention_implementation = "hip"

# options in the reference: ["torch", "triton", "cpp"]; this package: ["hip"]
gated_linear_unit_implementation = "hip"

# options in the reference: ["torch", "cpp"]; this package: ["hip"]
triangle_multiplication_implementation = "hip"

# Device weight caches are always on for "hip" (weights are cast/packed once per weight
# version); the reference's input-cache flags keep their meaning for the diffusion
# transformer's pair logits.
input_cache_enabled = False
packed_weight_cache_enabled = False
input_cache_max_bytes = 512 * 1024 * 1024

HIP = "hip"
