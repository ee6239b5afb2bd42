"""Parity of the MSA-stack operators (OuterProductMean, MSAAttention) and of EvoformerBlock
on the HIP backend against the CPU oracle (oracle/restatement.py), with the bars of
tests/test_gpu_ops.py: fp32 max error <= 1e-4 of RMS; bf16 RMS <= 2e-2 and max <= the
larger of 2e-2 and 1.5 x the case's bf16 floor.

Masks cover what the reference's modules meet: padded residues (whole mask columns zero,
xfold/nn/attention.py:132 then sends a key's logits to -1e9), padded sequences (mask rows
zero), ragged masks, fractional and boolean values."""

import pytest
import torch

from oracle import restatement as R
from tests.helpers import (TOL_FP32, assert_parity, assert_parity_bf16, bf16_stored, floor_of, load_fixture,
                           residual)
from tests.test_gpu_ops import announce, autocast, check_module, pair_of
from xfold_cpu_amd import nn as hnn
from xfold_cpu_amd.synthetic import init_module_

pytestmark = pytest.mark.gpu


def msa_mask(rows, n, seed, kind="ragged"):
    g = torch.Generator().manual_seed(seed)
    if kind == "ones":
        return torch.ones(rows, n)
    m = (torch.rand(rows, n, generator=g) > 0.2).float()
    m[-1, :] = 0                       # a padded sequence
    m[:, -2:] = 0                      # padded residues: no sequence covers them
    if kind == "fractional":
        m = m * torch.rand(rows, n, generator=g)
    if kind == "bool":
        m = m > 0
    return m


# ---------------------------------------------------------------------- OuterProductMean

@pytest.mark.parametrize("rows,n,c_msa,co,c_out", [(9, 37, 64, 32, 128), (1, 5, 16, 32, 32), (40, 70, 64, 16, 128),
                                                   (33, 64, 48, 8, 24)])
@pytest.mark.parametrize("bf16", [False, True])
def test_outer_product_mean(device, rows, n, c_msa, co, c_out, bf16):
    announce("outer_product_mean", rows, n, c_msa, co, c_out, bf16)
    ref, hip = pair_of("OuterProductMean", dict(c_msa=c_msa, num_output_channel=c_out, num_outer_channel=co),
                       seed=n)
    torch.manual_seed(n)
    msa = torch.randn(rows, n, c_msa)
    mask = msa_mask(rows, n, seed=n) if rows > 1 else torch.ones(rows, n)
    if bf16:
        msa = msa.bfloat16()
    check_module(ref, hip, hnn.outer_product_mean_hip, (msa.float(), mask), (msa.to(device), mask.to(device)),
                 bf16, "outer_product_mean")


@pytest.mark.parametrize("kind", ["ones", "fractional", "bool"])
def test_outer_product_mean_mask_values(device, kind):
    """All-ones, fractional and boolean masks (the norm divisor sums mask products)."""
    announce("outer_product_mean mask", kind)
    ref, hip = pair_of("OuterProductMean", dict(c_msa=64, num_output_channel=128, num_outer_channel=32), seed=3)
    torch.manual_seed(3)
    msa = torch.randn(21, 45, 64)
    mask = msa_mask(21, 45, seed=3, kind=kind)
    with torch.no_grad():
        want = ref(msa, mask.float())
    with torch.inference_mode():
        got = hip(msa.to(device), mask.to(device))
    assert_parity(got, want, TOL_FP32, f"outer_product_mean {kind} mask")


def test_outer_product_mean_at_trunk_size(device):
    """N = 256 residues, 192 sequences, bf16: the sequence reduction over several k-steps and
    the [N^2, 1024] output projection at a realistic shape."""
    announce("outer_product_mean trunk size")
    ref, hip = pair_of("OuterProductMean", dict(c_msa=64, num_output_channel=128, num_outer_channel=32), seed=11)
    torch.manual_seed(11)
    msa = torch.randn(192, 256, 64).bfloat16()
    mask = msa_mask(192, 256, seed=11)
    with torch.no_grad():
        want = ref(msa.float(), mask)
    floor = bf16_stored(floor_of(lambda: ref(msa.float(), mask)))
    with torch.inference_mode(), autocast(True):
        got = hip(msa.to(device), mask.to(device))
    assert_parity_bf16(got, want, "outer_product_mean N=256", floor=floor)


def test_outer_product_mean_rejects_empty_msa(device):
    _, hip = pair_of("OuterProductMean", dict(c_msa=16, num_output_channel=8, num_outer_channel=4), seed=1)
    with torch.inference_mode(), pytest.raises(ValueError, match="at least one MSA row"):
        hip(torch.randn(0, 5, 16, device=device), torch.ones(0, 5, device=device))


# -------------------------------------------------------------------------- MSAAttention

@pytest.mark.parametrize("rows,n,c_msa,c_pair,heads", [(5, 37, 64, 128, 8), (33, 200, 64, 128, 8),
                                                       (3, 50, 16, 32, 8), (7, 70, 64, 32, 4), (2, 3, 64, 128, 8)])
@pytest.mark.parametrize("bf16", [False, True])
def test_msa_attention(device, rows, n, c_msa, c_pair, heads, bf16):
    announce("msa_attention", rows, n, c_msa, c_pair, heads, bf16)
    ref, hip = pair_of("MSAAttention", dict(c_msa=c_msa, c_pair=c_pair, num_head=heads), seed=n)
    torch.manual_seed(n)
    msa = torch.randn(rows, n, c_msa)
    pair = torch.randn(n, n, c_pair)
    mask = msa_mask(rows, n, seed=n)
    if bf16:
        msa, pair = msa.bfloat16(), pair.bfloat16()
    check_module(ref, hip, hnn.msa_attention_hip, (msa.float(), mask, pair.float()),
                 (msa.to(device), mask.to(device), pair.to(device)), bf16, "msa_attention")


@pytest.mark.parametrize("kind", ["ones", "fractional", "bool"])
@pytest.mark.parametrize("c_pair", [128, 32])
def test_msa_attention_mask_values(device, kind, c_pair):
    announce("msa_attention mask", kind, c_pair)
    ref, hip = pair_of("MSAAttention", dict(c_msa=64, c_pair=c_pair, num_head=8), seed=4)
    torch.manual_seed(4)
    msa, pair = torch.randn(11, 66, 64), torch.randn(66, 66, c_pair)
    mask = msa_mask(11, 66, seed=4, kind=kind)
    with torch.no_grad():
        want = ref(msa, mask.float(), pair)
    with torch.inference_mode():
        got = hip(msa.to(device), mask.to(device), pair.to(device))
    assert_parity(got, want, TOL_FP32, f"msa_attention {kind} mask")


def test_msa_attention_fully_masked(device):
    """Every key masked: the reference's logits all get -1e9 and the softmax is uniform
    over the keys (fp32 cannot hold the -1e9-shifted logits' differences)."""
    announce("msa_attention fully masked")
    ref, hip = pair_of("MSAAttention", dict(c_msa=64, c_pair=128, num_head=8), seed=6)
    torch.manual_seed(6)
    msa, pair = torch.randn(4, 20, 64), torch.randn(20, 20, 128)
    mask = torch.zeros(4, 20)
    with torch.no_grad():
        want = ref(msa, mask, pair)
    with torch.inference_mode():
        got = hip(msa.to(device), mask.to(device), pair.to(device))
    assert torch.isfinite(got).all()
    assert_parity(got, want, TOL_FP32, "msa_attention fully masked")


# ------------------------------------------------------------------------- EvoformerBlock

def test_golden_evoformer_block(device):
    """fp32 golden vectors written by the reference's own EvoformerBlock."""
    announce("golden evoformer_block")
    meta, inputs, params, outputs = load_fixture("evoformer_block")
    module = hnn.EvoformerBlock(**meta["args"]).eval()
    module.load_state_dict(params, strict=True)
    module.to(device)
    d = {k: v.to(device) for k, v in inputs.items()}
    with torch.inference_mode():
        msa, pair = module(d["msa"].clone(), d["pair"].clone(), d["msa_mask"], d["pair_mask"])
    assert_parity(msa, outputs["msa"], TOL_FP32, "golden evoformer/msa")
    assert_parity(pair, outputs["pair"], TOL_FP32, "golden evoformer/pair")


@pytest.mark.parametrize("rows,n,mode", [(6, 24, "fp32"), (32, 64, "bf16"), (64, 130, "bf16")])
def test_evoformer_block(device, rows, n, mode):
    """The default-width block (c_msa 64, c_pair 128): fp32, and bf16 msa and pair updated in
    place (a bf16 residual stream, as the reference's model under autocast)."""
    announce("evoformer_block", rows, n, mode)
    ref, hip = pair_of("EvoformerBlock", dict(c_msa=64, c_pair=128, n_heads_pair=4), seed=n)
    torch.manual_seed(n)
    msa, pair = torch.randn(rows, n, 64), torch.randn(n, n, 128)
    mask = msa_mask(rows, n, seed=n)
    seq = torch.ones(n)
    seq[-2:] = 0
    pair_mask = seq[:, None] * seq[None, :]
    if mode == "bf16":
        msa, pair = msa.bfloat16(), pair.bfloat16()

    def oracle(wrap=lambda t: t):
        return ref(wrap(msa.float().clone()), wrap(pair.float().clone()), mask, pair_mask)
    with torch.no_grad():
        want_msa, want_pair = oracle()
    with torch.inference_mode(), autocast(mode == "bf16"):
        got_msa, got_pair = hip(msa.to(device).contiguous(), pair.to(device).contiguous(), mask.to(device),
                                pair_mask.to(device))
    if mode == "fp32":
        assert_parity(got_msa, want_msa, TOL_FP32, "evoformer msa")
        assert_parity(got_pair, want_pair, TOL_FP32, "evoformer pair")
        return
    floor_msa, floor_pair = floor_of(lambda: oracle(residual))
    assert got_pair.dtype == torch.bfloat16
    assert_parity_bf16(got_msa, want_msa, "evoformer msa", floor=floor_msa)
    assert_parity_bf16(got_pair, want_pair, "evoformer pair", floor=floor_pair)
