"""Edge sizes through the HIP modules and the attention entry point: one to three tokens,
single queries and keys, every mask rank the reference accepts
(xfold/fastnn/attention.py:57-62), against the oracle at the fp32 and bf16 bars."""

import pytest
import torch

from oracle import restatement as R
from tests.helpers import TOL_FP32, assert_parity, assert_parity_bf16, floor_of, residual
from tests.test_gpu_ops import announce, autocast, pair_of, run_both
from xfold_cpu_amd import fastnn

pytestmark = pytest.mark.gpu


def check(got, want, bf16, what, floor=None):
    assert torch.isfinite(got.float()).all(), what
    if bf16:
        assert_parity_bf16(got, want, what, floor=floor)
    else:
        assert_parity(got, want, TOL_FP32, what)


def pair_case(n, seed, masked_last=False):
    g = torch.Generator().manual_seed(seed)
    pair = torch.randn(n, n, 128, generator=g)
    seq = torch.ones(n)
    if masked_last:
        seq[-1] = 0
    return pair, seq[:, None] * seq[None, :]


@pytest.mark.parametrize("n,masked_last", [(1, False), (2, True), (3, False)])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("bf16", [False, True])
def test_triangle_multiplication_tiny(device, n, masked_last, outgoing, bf16):
    announce("trimul tiny", n, masked_last, outgoing, bf16)
    ref, hip = pair_of("TriangleMultiplication", dict(c_pair=128, _outgoing=outgoing), seed=n)
    pair, mask = pair_case(n, n, masked_last)
    if bf16:
        pair = pair.bfloat16()
    got, want = run_both(ref, hip, (pair.float(), mask), (pair.to(device), mask.to(device)), bf16)
    check(got, want, bf16, "trimul tiny", floor_of(lambda: ref(*(pair.float(), mask)), stored=True) if bf16 else None)


@pytest.mark.parametrize("n,masked_last", [(1, False), (2, True), (3, False)])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_grid_self_attention_tiny(device, n, masked_last, transpose, bf16):
    announce("grid attention tiny", n, masked_last, transpose, bf16)
    ref, hip = pair_of("GridSelfAttention", dict(c_pair=128, num_head=4, transpose=transpose), seed=n + 1)
    pair, mask = pair_case(n, n + 1, masked_last)
    if bf16:
        pair = pair.bfloat16()
    got, want = run_both(ref, hip, (pair.float(), mask), (pair.to(device), mask.to(device)), bf16)
    check(got, want, bf16, "grid attention tiny", floor_of(lambda: ref(*(pair.float(), mask)), stored=True) if bf16 else None)


@pytest.mark.parametrize("rows", [(1,), (1, 1), (3, 1)])
@pytest.mark.parametrize("bf16", [False, True])
def test_transition_tiny(device, rows, bf16):
    announce("transition tiny", rows, bf16)
    ref, hip = pair_of("Transition", dict(c_x=128, num_intermediate_factor=4), seed=5)
    x = torch.randn(*rows, 128)
    if bf16:
        x = x.bfloat16()
    got, want = run_both(ref, hip, (x.float(),), (x.to(device),), bf16)
    check(got, want, bf16, "transition tiny", floor_of(lambda: ref(*(x.float(),)), stored=True) if bf16 else None)


@pytest.mark.parametrize("q_len,k_len", [(1, 1), (1, 5), (4, 1), (2, 65)])
@pytest.mark.parametrize("mask_rank", [None, 1, 2, 4])
@pytest.mark.parametrize("d", [7, 24, 48])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attention_edge_shapes(device, q_len, k_len, mask_rank, d, dtype):
    """Single queries and keys, every mask rank of the reference's broadcast rules, batch-shared
    bias; masks keep the first key so that no row is fully masked."""
    announce("attention edges", q_len, k_len, mask_rank, d, dtype)
    g = torch.Generator().manual_seed(q_len * 100 + k_len + d)
    B, H = 2, 3
    q = torch.randn(B, H, q_len, d, generator=g).to(dtype)
    k = torch.randn(B, H, k_len, d, generator=g).to(dtype)
    v = torch.randn(B, H, k_len, d, generator=g).to(dtype)
    bias = torch.randn(H, q_len, k_len, generator=g).to(dtype)
    keep = torch.rand(B, k_len, generator=g) > 0.4
    keep[:, 0] = True
    mask = None if mask_rank is None else keep[0] if mask_rank == 1 else keep if mask_rank == 2 \
        else keep[:, None, None, :].expand(B, H, q_len, k_len).contiguous()
    def oracle():
        return R.dot_product_attention(q.float(), k.float(), v.float(), mask, bias.float())
    want, floor = oracle(), floor_of(oracle, stored=True)
    got = fastnn.dot_product_attention(q.to(device), k.to(device), v.to(device),
                                       None if mask is None else mask.to(device), bias.to(device))
    check(got, want, dtype == torch.bfloat16, "attention edges", floor)


@pytest.mark.parametrize("k_len,pipelined", [(4096, True), (4100, False)])
def test_attention_at_the_key_limit(device, k_len, pipelined):
    """bf16 attention at the pipelined kernel's key limit (4096 keys: 64 key blocks, the last
    one partly masked) and just beyond it, where the general kernel takes the call; the timer
    of the pipelined kernel tells which one ran."""
    from xfold_cpu_amd.fastnn import native_hip as nh
    announce("attention key limit", k_len)
    assert nh.attention_max_keys() == 4096
    g = torch.Generator().manual_seed(k_len)
    B, H, Q, d = 2, 2, 48, 32
    q, k, v = (torch.randn(B, H, n_, d, generator=g).bfloat16() for n_ in (Q, k_len, k_len))
    bias = torch.randn(H, Q, k_len, generator=g).bfloat16()
    keep = torch.rand(B, k_len, generator=g) > 0.3
    keep[:, 0] = True
    keep[:, -40:] = False
    def oracle():
        return R.dot_product_attention(q.float(), k.float(), v.float(), keep, bias.float())
    want, floor = oracle(), floor_of(oracle, stored=True)
    nh.kernel_timing_read("mha_attention")
    nh.set_kernel_timing(True)
    try:
        got = fastnn.dot_product_attention(q.to(device), k.to(device), v.to(device), keep.to(device),
                                           bias.to(device))
        torch.cuda.synchronize()
    finally:
        nh.set_kernel_timing(False)
    assert (nh.kernel_timing_read("mha_attention")[1] > 0) == pipelined
    check(got, want, True, f"attention {k_len} keys", floor)


@pytest.mark.parametrize("n,samples", [(1, 1), (2, 3), (5, 1)])
def test_diffusion_transformer_tiny(device, n, samples):
    announce("diffusion transformer tiny", n, samples)
    args = dict(c_act=256, c_single_cond=64, c_pair_cond=128, num_head=16, num_blocks=2, super_block_size=2)
    ref, hip = pair_of("DiffusionTransformer", args, seed=n + samples, device=device)
    g = torch.Generator().manual_seed(n)
    act = torch.randn(samples, n, 256, generator=g).bfloat16()
    mask = torch.ones(n)
    scond, pcond = torch.randn(n, 64, generator=g), torch.randn(n, n, 128, generator=g)
    def oracle(wrap=lambda t: t):
        return torch.stack([ref(wrap(act[s].float().clone()), mask, scond, pcond) for s in range(samples)])
    with torch.inference_mode():
        want = oracle()
        with autocast(True):
            got = hip(act.to(device).clone(), mask.to(device), scond.to(device), pcond.to(device))
    assert torch.isfinite(got.float()).all()
    assert_parity_bf16(got, want, "diffusion transformer tiny", floor=floor_of(lambda: oracle(residual)))


@pytest.mark.parametrize("module", ["TriangleMultiplication", "GridSelfAttention", "Transition"])
def test_strided_inputs(device, module):
    """Transposed (non-contiguous) pair and mask views give the result of their contiguous
    copies."""
    announce("strided inputs", module)
    args = {"TriangleMultiplication": dict(c_pair=128, _outgoing=False),
            "GridSelfAttention": dict(c_pair=128, num_head=4, transpose=True),
            "Transition": dict(c_x=128, num_intermediate_factor=4)}[module]
    ref, hip = pair_of(module, args, seed=9)
    n = 37
    g = torch.Generator().manual_seed(9)
    base = torch.randn(n, n, 128, generator=g).bfloat16()
    keep = (torch.rand(n, n, generator=g) > 0.2).float()
    pair, mask = base.transpose(0, 1), keep.t()
    dpair, dmask = base.to(device).transpose(0, 1), keep.to(device).t()
    assert not dpair.is_contiguous() and not dmask.is_contiguous()
    if module == "Transition":
        ref_in, dev_in = (pair.float(),), (dpair,)
    else:
        ref_in, dev_in = (pair.float(), mask), (dpair, dmask)
    got, want = run_both(ref, hip, ref_in, dev_in, True)
    check(got, want, True, f"{module} strided", floor_of(lambda: ref(*ref_in), stored=True))
