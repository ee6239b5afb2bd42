"""Parity of the atom CrossAttention (xfold/nn/diffusion_transformer.py:275-350) on the HIP
backend against the CPU oracle, with the bars of tests/test_gpu_ops.py (fp32: max error <=
1e-4 of RMS; bf16: RMS <= 2e-2 and max <= max(2e-2, 1.5 x the bf16 floor)).

Shapes follow the atom cross-attention of AF3 (query subsets of 32 atoms over 128 keys,
key_dim = value_dim = c_single_cond = 128, 4 heads): masked queries (which attend to the
masked keys only, through the reference's positive 1e9 term), masked keys, pair logits
shared per subset or absent."""

import pytest
import torch

from tests.helpers import TOL_FP32, assert_parity
from tests.test_gpu_ops import announce, check_module, pair_of

from xfold_cpu_amd import nn as hnn

pytestmark = pytest.mark.gpu


def cross_inputs(subsets, nq, nk, c, heads, seed, with_pair=True, lead=()):
    g = torch.Generator().manual_seed(seed)
    shape = lead + (subsets,)
    x_q, x_k = torch.randn(*shape, nq, c, generator=g), torch.randn(*shape, nk, c, generator=g)
    cond_q, cond_k = torch.randn(*shape, nq, c, generator=g), torch.randn(*shape, nk, c, generator=g)
    mask_q = (torch.rand(*shape, nq, generator=g) > 0.1).float()
    mask_k = (torch.rand(*shape, nk, generator=g) > 0.15).float()
    mask_q[..., 0, -1] = 0.0                            # a masked query in the first subset
    mask_k[..., 0, :3] = 0.0                            # ... which attends to these keys only
    pair = torch.randn(*shape, heads, nq, nk, generator=g) if with_pair else None
    return x_q, x_k, mask_q, mask_k, pair, cond_q, cond_k


@pytest.mark.parametrize("subsets,nq,nk,c,heads", [(24, 32, 128, 128, 4), (3, 5, 7, 32, 4), (2, 32, 100, 64, 2)])
@pytest.mark.parametrize("with_pair", [True, False])
@pytest.mark.parametrize("bf16", [False, True])
def test_cross_attention(device, subsets, nq, nk, c, heads, with_pair, bf16):
    announce("cross_attention", subsets, nq, nk, c, heads, with_pair, bf16)
    args = dict(key_dim=c, value_dim=c, c_single_cond=c, num_head=heads)
    ref, hip = pair_of("CrossAttention", args, seed=subsets + nk)
    x_q, x_k, mask_q, mask_k, pair, cond_q, cond_k = cross_inputs(subsets, nq, nk, c, heads, seed=nk,
                                                                  with_pair=with_pair)
    if bf16:
        x_q, x_k, cond_q, cond_k = (t.bfloat16() for t in (x_q, x_k, cond_q, cond_k))
        pair = pair.bfloat16() if pair is not None else None
    f32 = lambda t: None if t is None else t.float()
    dev = lambda t: None if t is None else t.to(device)
    check_module(ref, hip, hnn.cross_attention_hip,
                 (f32(x_q), f32(x_k), mask_q, mask_k, f32(pair), f32(cond_q), f32(cond_k)),
                 tuple(dev(t) for t in (x_q, x_k, mask_q, mask_k, pair, cond_q, cond_k)), bf16, "cross_attention")


def test_cross_attention_broadcast_pair_logits_and_bool_masks(device):
    """Leading batch dims, pair logits broadcast over them, boolean masks."""
    announce("cross_attention broadcast")
    args = dict(key_dim=64, value_dim=64, c_single_cond=64, num_head=4)
    ref, hip = pair_of("CrossAttention", args, seed=5)
    x_q, x_k, mask_q, mask_k, _, cond_q, cond_k = cross_inputs(6, 16, 40, 64, 4, seed=5, lead=(2,))
    pair = torch.randn(6, 4, 16, 40)
    with torch.no_grad():
        want = ref(x_q, x_k, mask_q, mask_k, pair, cond_q, cond_k)
    with torch.inference_mode():
        got = hip(*(t.to(device) for t in (x_q, x_k, mask_q > 0, mask_k > 0, pair, cond_q, cond_k)))
    assert_parity(got, want, TOL_FP32, "cross_attention broadcast")
