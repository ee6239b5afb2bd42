"""Parity at the benchmark sizes: one bf16 Pairformer pair block at N=768 with 77 padded
tokens (the C3 trunk's block, xfold/nn/pairformer.py:77-114) and one bf16 outgoing triangle
multiplication at N=1536 (the C5 size, xfold/nn/triangle_multiplication.py:71-105), each
against the fp32 CPU oracle on the same bf16 inputs (the oracle's attention in row chunks, so
that its logits stay small). Each oracle run takes 15-35 s of host time."""

import pytest
import torch

from oracle import restatement as R
from tests.helpers import assert_parity_bf16
from tests.test_gpu_ops import announce, autocast, pair_of
from xfold_cpu_amd.synthetic import pair_block_inputs

pytestmark = pytest.mark.gpu


def chunked_attention(*args, **kwargs):
    return R.dot_product_attention_chunked(*args, rows_per_chunk=32, **kwargs)


def test_pair_block_n768(device):
    n = 768
    announce("full size pair block", n)
    args = dict(n_heads=16, c_pair=128, c_single=384, n_heads_pair=4, with_single=False)
    ref, hip = pair_of("PairformerBlock", args, seed=48, device=device)
    inp = pair_block_inputs(n, pad=77, seed=48, with_single=False)
    pair = inp.pair.bfloat16()
    with torch.inference_mode():
        with autocast(True):
            got = hip(pair.to(device).contiguous(), inp.pair_mask.to(device))
        got = got.float().cpu()
        want = ref(pair.float(), inp.pair_mask, attention=chunked_attention)
    assert torch.isfinite(got).all()
    # bf16 residual stream, rounded at each of its 5 in-place updates.
    assert_parity_bf16(got, want, "pair block N=768", stores=5)


def test_triangle_multiplication_n1536(device):
    n = 1536
    announce("full size trimul", n)
    ref, hip = pair_of("TriangleMultiplication", dict(c_pair=128, _outgoing=True), seed=15)
    g = torch.Generator().manual_seed(15)
    pair = torch.randn(n, n, 128, generator=g).bfloat16()
    seq = torch.ones(n)
    seq[torch.randperm(n, generator=g)[:77]] = 0          # C5: 5% of the tokens padded at random
    mask = seq[:, None] * seq[None, :]
    with torch.inference_mode():
        with autocast(True):
            got = hip(pair.to(device), mask.to(device))
        got = got.float().cpu()
        want = ref(pair.float(), mask)
    assert torch.isfinite(got).all()
    assert_parity_bf16(got, want, "trimul N=1536")
