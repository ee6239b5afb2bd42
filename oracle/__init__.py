"""Test infrastructure: the CPU oracle for the Pairformer / diffusion-transformer path.

THIS PACKAGE IS NOT PRODUCT CODE. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker (or, for the
CPU baseline, as the thing timed on the host). Nothing under ``xfold_cpu_amd/`` imports it.

Contents
--------
``restatement``  A PyTorch-on-CPU restatement of the reference's ``torch`` backend for every
                 operator on the hot path (LayerNorm, GLU, dot-product attention, triangle
                 multiplication, grid self-attention, transitions, adaptive LayerNorm, the
                 single-track / diffusion SelfAttention, PairformerBlock and the diffusion
                 transformer). Each function cites the reference file:line it follows. The
                 modules keep the reference's parameter names so one ``state_dict`` loads into
                 the oracle and into the HIP modules alike.
``brute``        Pure-Python loop versions of LayerNorm, attention and triangle multiplication
                 for tiny shapes. They pin the restatement independently of ATen's kernels.

How each oracle function is pinned (a function without a pin says "parity unpinned"):
  layer_norm                 closed form (mean/var/rstd) + ``brute.layer_norm`` + the reference
                             test's exact comparison with ``F.layer_norm``
                             (tests/test_cpu_runtime.py:52-60 in the reference).
  gated_linear_unit          closed form ``silu(x@Wg) * (x@Wv)`` with the first half as the gate
                             (reference tests/test_cpu_runtime.py:62-68).
  dot_product_attention      einsum restatement with -1e9 fill, mask ranks 1/2/4 (reference
                             tests/test_cpu_runtime.py:70-89), ``brute.attention``, uniform
                             softmax on a fully masked row, and SDPA with no bias/mask.
  TriangleMultiplication     explicit per-channel matmul with the even/odd channel split in
                             both directions (reference tests/test_cpu_runtime.py:104-115),
                             ``brute.triangle_multiplication``, and golden vectors.
  GridSelfAttention, Transition, SelfAttention (with and without conditioning),
  DiffusionTransition, PairformerBlock, DiffusionTransformer
                             golden vectors written by ``tests/golden/make_golden.py`` from the
                             reference modules themselves (fp32 and CPU bf16 autocast).
"""
