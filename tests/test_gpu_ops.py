"""Per-operator parity of the HIP backend against the CPU oracle (oracle/restatement.py).

Bars, relative to RMS(oracle):
  * fp32 mode: max |hip - oracle| <= 1e-4 (TOL_FP32).
  * bf16 mode (CUDA bf16 autocast: bf16 operands, fp32 accumulation): RMS error <= 2e-2
    (TOL_BF16) and max error <= max(2e-2, 1.5 x the case's bf16 floor), against the oracle
    run in fp32 on the same bf16-rounded inputs and fp32 weights; the floor is the same
    oracle evaluation with bf16-rounded matrix-product operands, and a bf16-stored output
    rounded once (see tests/helpers.py). Module outputs are checked both as stored (bf16,
    their dtype contract) and accumulated into fp32.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import restatement as R
from tests.helpers import (TOL_BF16, TOL_FP32, assert_parity, assert_parity_bf16, bf16_stored, floor_of,
                           rel_err)
from xfold_cpu_amd import fastnn
from xfold_cpu_amd import nn as hnn
from xfold_cpu_amd.fastnn import native_hip as nh
from xfold_cpu_amd.fastnn import ops
from xfold_cpu_amd.synthetic import init_module_

pytestmark = pytest.mark.gpu


def announce(*what):
    print("[case]", *what, flush=True)


def pair_of(cls_name, args, seed=0, device="cuda"):
    """(oracle module on CPU fp32, HIP module on device) with identical jittered weights."""
    ref = init_module_(getattr(R, cls_name)(**args).eval(), seed=seed, ln_jitter=True)
    hip = getattr(hnn, cls_name)(**args).eval()
    hip.load_state_dict(ref.state_dict())
    return ref, hip.to(device)


def autocast(enabled):
    return torch.amp.autocast("cuda", dtype=torch.bfloat16, enabled=enabled)


# ---------------------------------------------------------------------------- LayerNorm

@pytest.mark.parametrize("cols", [128, 384, 768, 7, 100])
@pytest.mark.parametrize("dt_in,dt_out", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("affine", ["full", "weight", "none"])
def test_layer_norm(device, cols, dt_in, dt_out, affine):
    announce("layer_norm", cols, dt_in, dt_out, affine)
    torch.manual_seed(cols)
    x = (torch.randn(301, cols) * 3 + 1).to(dt_in)
    w = torch.randn(cols) if affine != "none" else None
    b = torch.randn(cols) if affine == "full" else None
    want = F.layer_norm(x.float(), (cols,), w, b, 1e-5)
    got = ops.layer_norm(x.to(device), (cols,), None if w is None else w.to(device),
                         None if b is None else b.to(device), 1e-5, out_dtype=dt_out)
    assert got.dtype == dt_out
    if dt_out == torch.bfloat16:
        assert_parity_bf16(got, want, "layer_norm", floor=bf16_stored(want))
    else:
        # bf16 inputs are exact in fp32, so the fp32-output kernel meets the fp32 bar.
        want = F.layer_norm(x.float(), (cols,), w, b, 1e-5)
        assert_parity(got, want, TOL_FP32, "layer_norm")


@pytest.mark.parametrize("dt_in,dt_out", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                          (torch.float32, torch.bfloat16)])
def test_layer_norm_many_rows(device, dt_in, dt_out):
    """Pair-sized row counts (several rows per lane group), not a multiple of 4 rows."""
    announce("layer_norm many rows", dt_in, dt_out)
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(70001, 128, generator=g) * 2 - 0.5).to(dt_in)
    w, b = torch.randn(128, generator=g), torch.randn(128, generator=g)
    want = F.layer_norm(x.float(), (128,), w, b, 1e-5)
    got = ops.layer_norm(x.to(device), (128,), w.to(device), b.to(device), 1e-5, out_dtype=dt_out)
    if dt_out == torch.bfloat16:
        assert_parity_bf16(got, want, "layer_norm many rows", floor=bf16_stored(want))
    else:
        assert_parity(got, want, TOL_FP32, "layer_norm many rows")


def test_layer_norm_module_dtype_contract(device):
    ln = fastnn.LayerNorm(128).eval().to(device)
    x = torch.randn(4, 128, device=device, dtype=torch.bfloat16)
    with torch.inference_mode():
        assert ln(x).dtype == torch.bfloat16
        with autocast(True):
            assert ln(x).dtype == torch.float32        # CUDA autocast runs layer_norm in fp32
        assert ln(x.float()).dtype == torch.float32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adaptive_layer_norm(device, dtype):
    announce("adaptive_layer_norm", dtype)
    torch.manual_seed(1)
    x = torch.randn(3, 40, 768).to(dtype)
    scale, shift = torch.randn(40, 768).to(dtype), torch.randn(40, 768).to(dtype)
    want = torch.sigmoid(scale.float()) * F.layer_norm(x.float(), (768,)) + shift.float()
    got = ops.adaptive_layer_norm(x.to(device), scale.to(device), shift.to(device), 1e-5, torch.float32)
    assert_parity(got, want, TOL_FP32, "adaptive_ln")
    got = ops.adaptive_layer_norm(x.to(device), scale.to(device), shift.to(device), 1e-5, dtype)
    if dtype == torch.bfloat16:
        assert_parity_bf16(got, want, "adaptive_ln bf16 store", floor=bf16_stored(want))


# ---------------------------------------------------------------------------- Linear / GLU

@pytest.mark.parametrize("m,k,n", [(1, 7, 5), (77, 128, 128), (300, 384, 200), (129, 96, 257)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("epi", [nh.EPI_STORE, nh.EPI_MUL_SIGMOID_AUX, nh.EPI_SIGMOID_MUL_AUX,
                                 nh.EPI_ACCUMULATE, nh.EPI_MUL_SIGMOID_AUX_ACCUMULATE])
def test_linear_epilogues(device, m, k, n, dtype, epi):
    announce("linear", m, k, n, dtype, epi)
    torch.manual_seed(m + k + n)
    x = torch.randn(m, k).to(dtype)
    w = (torch.randn(n, k) / math.sqrt(k)).to(dtype)
    bias = torch.randn(n)
    aux = torch.randn(m, n).to(dtype)
    c0 = torch.randn(m, n).to(dtype)
    acc = x.float() @ w.float().T + bias
    want = {nh.EPI_STORE: acc, nh.EPI_MUL_SIGMOID_AUX: acc * torch.sigmoid(aux.float()),
            nh.EPI_SIGMOID_MUL_AUX: torch.sigmoid(acc) * aux.float(),
            nh.EPI_ACCUMULATE: c0.float() + acc,
            nh.EPI_MUL_SIGMOID_AUX_ACCUMULATE: c0.float() + acc * torch.sigmoid(aux.float())}[epi]
    out = c0.to(device).clone()
    needs_aux = epi in (nh.EPI_MUL_SIGMOID_AUX, nh.EPI_SIGMOID_MUL_AUX, nh.EPI_MUL_SIGMOID_AUX_ACCUMULATE)
    ops.linear(x.to(device), w.to(device), bias.to(device), dtype, out=out, epilogue=epi,
               aux=aux.to(device) if needs_aux else None)
    if dtype == torch.float32:
        assert_parity(out, want, TOL_FP32, "linear")
    else:
        assert_parity_bf16(out, want, "linear bf16 store", floor=bf16_stored(want))
        out32 = c0.float().to(device).clone()
        ops.linear(x.to(device), w.to(device), bias.to(device), dtype, out=out32, epilogue=epi,
                   aux=aux.float().to(device) if needs_aux else None)
        assert_parity_bf16(out32, want, "linear bf16 compute, fp32 out")


@pytest.mark.parametrize("m,k,n,nb", [(77, 384, 768, 6), (5, 64, 40, 3), (300, 96, 130, 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shared", [True, False])
@pytest.mark.parametrize("with_bias", [True, False])
def test_linear_batched(device, m, k, n, nb, dtype, shared, with_bias):
    """One launch over B weight matrices (and biases), with one shared input or B inputs."""
    announce("linear_batched", m, k, n, nb, dtype, shared, with_bias)
    torch.manual_seed(m + n + nb)
    x = torch.randn(m, k) if shared else torch.randn(nb, m, k)
    x = x.to(dtype)
    w = (torch.randn(nb, n, k) / math.sqrt(k)).to(dtype)
    bias = torch.randn(nb, n) if with_bias else None
    want = torch.einsum("mk,bnk->bmn" if shared else "bmk,bnk->bmn", x.float(), w.float())
    if with_bias:
        want = want + bias[:, None, :]
    got = ops.linear_batched(x.to(device), w.to(device), None if bias is None else bias.to(device), dtype)
    assert got.shape == (nb, m, n) and got.dtype == dtype
    if dtype == torch.float32:
        assert_parity(got, want, TOL_FP32, "linear_batched")
    else:
        assert_parity_bf16(got, want, "linear_batched", floor=bf16_stored(want))


def test_linear_aux_rows_broadcast(device):
    torch.manual_seed(2)
    x, w, aux = torch.randn(3, 10, 64), torch.randn(32, 64) / 8, torch.randn(10, 32)
    want = (x @ w.T) * torch.sigmoid(aux)
    got = ops.linear(x.to(device), w.to(device), None, torch.float32, epilogue=nh.EPI_MUL_SIGMOID_AUX,
                     aux=aux.to(device), aux_rows=10)
    assert_parity(got, want, TOL_FP32, "aux rows")


@pytest.mark.parametrize("m,k,f", [(6, 7, 5), (1000, 128, 512), (333, 384, 1536), (50, 768, 1536)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_linear_unit(device, m, k, f, dtype):
    announce("glu", m, k, f, dtype)
    torch.manual_seed(k)
    x = torch.randn(m, k).to(dtype)
    weight = (torch.randn(2 * f, k) / math.sqrt(k)).T.to(dtype)      # [K, 2F] like transition1.weight.T
    want = R.gated_linear_unit(x.float(), weight.float())
    got = fastnn.gated_linear_unit(x.to(device), weight.to(device))
    if dtype == torch.float32:
        assert_parity(got, want, TOL_FP32, "glu")
        return
    assert_parity_bf16(got, want, "glu bf16 store", floor=bf16_stored(want))
    packed = nh._prepare(weight.T.to(device), dtype, "glu")
    got32 = ops.gated_linear_unit(x.to(device), packed, f, dtype, out_dtype=torch.float32)
    assert_parity_bf16(got32, want, "glu bf16 compute, fp32 out")


# ---------------------------------------------------------------------------- attention

@pytest.mark.parametrize("n,heads", [(70, 16), (33, 20), (128, 384)])
@pytest.mark.parametrize("pair_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_pair_attention_bias(device, n, heads, pair_dtype, out_dtype):
    """Linear(LayerNorm(pair)) rearranged to [h, i, j] in the packed layout with zero pad
    columns (xfold/nn/pairformer.py:103-106): fp32 times log2(e), or bf16 logits."""
    announce("pair_attention_bias", n, heads, pair_dtype, out_dtype)
    g = torch.Generator().manual_seed(n + heads)
    pair = (torch.randn(n, n, 128, generator=g) * 2 + 0.5).to(pair_dtype)
    ln_w, ln_b = 1 + 0.1 * torch.randn(128, generator=g), 0.1 * torch.randn(128, generator=g)
    w = (torch.randn(heads, 128, generator=g) / math.sqrt(128)).bfloat16()
    scale = math.log2(math.e) if out_dtype == torch.float32 else 1.0
    def oracle():
        out = F.layer_norm(pair.float(), (128,), ln_w, ln_b, 1e-5) @ w.float().T
        return out.permute(2, 0, 1) * scale
    want, floor = oracle(), floor_of(oracle)
    got = ops.pair_attention_bias(pair.to(device), ln_w.to(device), ln_b.to(device), 1e-5, w.to(device),
                                  out_dtype=out_dtype)
    npad = (n + 63) // 64 * 64
    assert got.shape == (heads, n, npad) and got.dtype == out_dtype
    assert bool((got[..., n:] == 0).all())
    if out_dtype == torch.bfloat16:
        floor = bf16_stored(floor)
    assert_parity_bf16(got[..., :n], want, "pair_attention_bias", floor=floor)


@pytest.mark.parametrize("n,heads", [(1, 16), (37, 16), (64, 4), (130, 16), (257, 7)])
def test_transition_pair_bias_fused(device, n, heads):
    """The single-track block's pair transition with the pair logits computed in its epilogue
    (xfh_transition_pair_bias) equals xfh_transition then xfh_pair_attention_bias bit for
    bit: the updated pair, the packed logits and their zero pad columns (xfold/nn/pairformer.py:100-106)."""
    from xfold_cpu_amd.nn import pairformer as P
    from xfold_cpu_amd.nn.primitives import transition_hip
    announce("transition_pair_bias", n, heads)
    ref = init_module_(R.PairformerBlock(n_heads=heads, with_single=True).eval(), seed=n, ln_jitter=True)
    block = hnn.PairformerBlock(n_heads=heads, with_single=True).eval()
    block.load_state_dict(ref.state_dict())
    block = block.to(device)
    g = torch.Generator().manual_seed(n + 3 * heads)
    pair = (torch.randn(n, n, 128, generator=g) * 2 + 0.5).bfloat16().to(device)
    fused, split = pair.clone(), pair.clone()
    with torch.inference_mode(), torch.amp.autocast("cuda", dtype=torch.bfloat16):
        got = P._transition_with_logits_hip(block, fused)
        transition_hip(block.pair_transition, split, accumulate_into=split)
        norm = block.single_pair_logits_norm
        want = ops.pair_attention_bias(split, norm.weight, norm.bias, norm.eps,
                                       nh.linear_weight(block, "single_pair_logits_projection", torch.bfloat16),
                                       owner=norm)
    torch.cuda.synchronize()
    assert got is not None and got.tensor.shape == want.shape == (heads, n, (n + 63) // 64 * 64)
    assert torch.equal(fused, split), "updated pair differs"
    assert torch.equal(got.tensor, want), f"logits differ: max {(got.tensor - want).abs().max().item()}"
    assert bool((got.tensor[..., n:] == 0).all())


@pytest.mark.parametrize("d", [32, 48, 64])
@pytest.mark.parametrize("batch", [1, 3])
def test_attention_packed_bias_bf16(device, d, batch):
    """A bf16 packed bias (natural units, widened and scaled by log2(e) in the kernel) gives
    the same bits as the fp32 packed bias of the same bf16 logits."""
    announce("attention packed bias bf16", d, batch)
    g = torch.Generator().manual_seed(d + batch)
    H, N = 4, 100
    npad = 128
    q, k, v = (torch.randn(batch, H, N, d, generator=g).bfloat16().to(device) for _ in range(3))
    mask = (torch.rand(batch, N, generator=g) > 0.2).to(device)
    logits = (torch.randn(H, N, N, generator=g) * 3).bfloat16().to(device)
    packed32 = ops.PackedBias(ops.attention_bias_pack(logits[None])[0])
    packed16 = ops.PackedBias(F.pad(logits, (0, npad - N)).contiguous())
    assert packed16.code == nh.BIAS_PACKED_BF16
    want = ops.attention(q, k, v, mask, packed32)
    got = ops.attention(q, k, v, mask, packed16)
    assert torch.equal(got, want), f"max diff {(got.float() - want.float()).abs().max().item()}"


@pytest.mark.parametrize("d", [32, 48, 64])
@pytest.mark.parametrize("head_minor", [True, False])
def test_attention_packed_bias(device, d, head_minor):
    """A bias converted once by attention_bias_pack (head-minor bf16 logits, as the
    diffusion transformer's super-block, or strided fp32) gives bit-identical attention to
    passing the same bias per call."""
    announce("attention packed bias", d, head_minor)
    g = torch.Generator().manual_seed(d)
    B, H, N, G = 3, 4, 100, 2
    q, k, v = (torch.randn(B, H, N, d, generator=g).bfloat16().to(device) for _ in range(3))
    mask = (torch.rand(B, N, generator=g) > 0.2).to(device)
    mask[1] = False                                   # a fully masked batch entry
    if head_minor:
        logits = torch.randn(N, N, G * H, generator=g).bfloat16().to(device)
        biases = logits.view(N, N, G, H).permute(2, 3, 0, 1)
    else:
        biases = torch.randn(G, H, N, N, generator=g).to(device)
    packed = ops.attention_bias_pack(biases)
    assert packed.shape == (G, H, N, 128) and bool((packed[..., N:] == 0).all())
    for j in range(G):
        want = ops.attention(q, k, v, mask, biases[j])
        got = ops.attention(q, k, v, mask, ops.PackedBias(packed[j]))
        assert torch.equal(got, want), f"block {j}: max diff {(got.float() - want.float()).abs().max().item()}"


@pytest.mark.parametrize("mask_rank", [1, 2, 4])
@pytest.mark.parametrize("batched", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attention_reference_cases(device, mask_rank, batched, dtype):
    """The reference's own attention case (tests/test_cpu_runtime.py:70-89): odd head dim 7."""
    torch.manual_seed(42)
    q, k, v = [torch.randn(*s).to(dtype) for s in ((1, 2, 3, 7), (1, 2, 5, 7), (1, 2, 5, 4))]
    mask = torch.tensor([1, 1, 0, 1, 0], dtype=torch.bool)
    expanded = mask[None, None, None, :]
    passed = mask if mask_rank == 1 else mask[None] if mask_rank == 2 else expanded
    bias = torch.randn(1, 2, 3, 5).to(dtype)
    def oracle():
        return R.dot_product_attention(q.float(), k.float(), v.float(), passed, bias.float())
    want, floor = oracle(), floor_of(oracle)
    if not batched:
        q, k, v, bias, want, floor = q[0], k[0], v[0], bias[0], want[0], floor[0]
    got = fastnn.dot_product_attention(q.to(device), k.to(device), v.to(device), passed.to(device),
                                       bias.to(device))
    if dtype == torch.float32:
        assert_parity(got, want, TOL_FP32, "attention")
    else:
        assert_parity_bf16(got, want, "attention bf16 store", floor=bf16_stored(floor))


@pytest.mark.parametrize("shape", [(3, 4, 37, 37, 32), (1, 16, 100, 100, 24), (2, 16, 70, 70, 48),
                                   (2, 3, 65, 130, 64), (1, 1, 1, 1, 16), (1, 4, 50, 77, 16),
                                   (5, 2, 33, 70, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attention_shapes_masks_and_fully_masked_rows(device, shape, dtype):
    B, H, Q, K, D = shape
    announce("attention", shape, dtype)
    torch.manual_seed(Q + K)
    q, k, v = torch.randn(B, H, Q, D).to(dtype), torch.randn(B, H, K, D).to(dtype), torch.randn(B, H, K, D).to(dtype)
    bias = torch.randn(H, Q, K).to(dtype)
    mask = torch.rand(B, K) > 0.25
    mask[0] = False                      # a fully masked batch row: uniform average of v
    def oracle():
        return R.dot_product_attention(q.float(), k.float(), v.float(), mask, bias.float())
    want, floor = oracle(), floor_of(oracle)
    dq, dk, dv = q.to(device), k.to(device), v.to(device)
    got = fastnn.dot_product_attention(dq, dk, dv, mask.to(device), bias.to(device))
    uniform = v[0].float().mean(1, keepdim=True).expand(H, Q, D)
    if dtype == torch.float32:
        assert_parity(got, want, TOL_FP32, "attention")
        assert_parity(got[0], uniform, TOL_FP32, "uniform row")
        return
    assert_parity_bf16(got, want, "attention bf16 store", floor=bf16_stored(floor))
    got32 = ops.attention(dq, dk, dv, mask.to(device), bias.to(device), out_dtype=torch.float32)
    assert_parity_bf16(got32, want, "attention bf16 compute, fp32 out", floor=floor)
    assert_parity_bf16(got32[0], uniform, "uniform row")


def test_attention_float_mask_and_no_bias(device):
    torch.manual_seed(3)
    q, k, v = torch.randn(2, 2, 9, 16), torch.randn(2, 2, 11, 16), torch.randn(2, 2, 11, 16)
    mask = (torch.rand(2, 11) > 0.5).float()
    want = R.dot_product_attention(q, k, v, mask, None)
    got = fastnn.dot_product_attention(q.to(device), k.to(device), v.to(device), mask.to(device), None)
    assert_parity(got, want, TOL_FP32, "float mask")
    want = F.scaled_dot_product_attention(q, k, v)
    got = fastnn.dot_product_attention(q.to(device), k.to(device), v.to(device))
    assert_parity(got, want, TOL_FP32, "sdpa")


# ---------------------------------------------------------------------------- modules

def run_both(ref, hip, ref_inputs, dev_inputs, bf16, call=None):
    call = call or (lambda m, *a: m(*a))
    with torch.inference_mode():
        want = call(ref, *ref_inputs)
        with autocast(bf16):
            got = call(hip, *dev_inputs)
    return got, want


def check_module(ref, hip, hip_fn, ref_inputs, dev_inputs, bf16, what):
    """fp32: module output vs oracle at 1e-4. bf16: the module's bf16 output and the same
    op accumulated into an fp32 zero tensor, both at the bf16 bar, the max error against
    the bf16-operand floor of the same oracle call."""
    got, want = run_both(ref, hip, ref_inputs, dev_inputs, bf16)
    if not bf16:
        assert got.dtype == torch.float32
        return assert_parity(got, want, TOL_FP32, what)
    assert got.dtype == torch.bfloat16
    floor = floor_of(lambda: ref(*ref_inputs))
    assert_parity_bf16(got, want, what + " (bf16 store)", floor=bf16_stored(floor))
    out32 = torch.zeros(got.shape, dtype=torch.float32, device=got.device)
    with torch.inference_mode(), autocast(True):
        hip_fn(hip, *dev_inputs, accumulate_into=out32)
    return assert_parity_bf16(out32, want, what + " (bf16 compute, fp32 out)", floor=floor)


@pytest.mark.parametrize("n", [5, 37, 64, 200])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("bf16", [False, True])
def test_triangle_multiplication(device, n, outgoing, bf16):
    announce("trimul", n, outgoing, bf16)
    ref, hip = pair_of("TriangleMultiplication", dict(c_pair=128, _outgoing=outgoing), seed=n)
    torch.manual_seed(n)
    pair = torch.randn(n, n, 128)
    seq = torch.ones(n)
    seq[-2:] = 0
    mask = seq[:, None] * seq[None, :]
    if bf16:
        pair = pair.bfloat16()
    check_module(ref, hip, hnn.triangle_multiplication_hip, (pair.float(), mask),
                 (pair.to(device), mask.to(device)), bf16, "trimul")


@pytest.mark.parametrize("c,n", [(64, 40), (96, 33), (288, 24)])
@pytest.mark.parametrize("bf16", [False, True])
def test_triangle_multiplication_other_widths(device, c, n, bf16):
    """Pair widths off the c = 128 fast path (the generic GEMM and LayerNorm kernels): the
    template stack's 64, an odd multiple of 32, and 288 (> 256 channels, where the
    channel-plane LayerNorm takes its untiled form)."""
    announce("trimul width", c, n, bf16)
    ref, hip = pair_of("TriangleMultiplication", dict(c_pair=c, _outgoing=True), seed=c + n)
    torch.manual_seed(c)
    pair = torch.randn(n, n, c)
    seq = torch.ones(n)
    seq[-3:] = 0
    mask = seq[:, None] * seq[None, :]
    if bf16:
        pair = pair.bfloat16()
    check_module(ref, hip, hnn.triangle_multiplication_hip, (pair.float(), mask),
                 (pair.to(device), mask.to(device)), bf16, f"trimul c={c}")


# n = 520: enough 32-position units (520 x 17) for the 32-position projection path on a
# 256-CU device; the smaller sizes take the 16-position path.
@pytest.mark.parametrize("n,mask_dtype", [(33, torch.float32), (96, torch.bfloat16), (45, torch.bool),
                                          (520, torch.float32)])
@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_mask_values(device, n, mask_dtype, outgoing):
    """Fractional (float, bf16) and boolean masks, asymmetric, on sizes with and without pad
    columns in the contraction operands: the mask scales every projected channel of its
    position, in the orientation the module reads it."""
    announce("trimul mask", n, mask_dtype, outgoing)
    ref, hip = pair_of("TriangleMultiplication", dict(c_pair=128, _outgoing=outgoing), seed=n + 7)
    g = torch.Generator().manual_seed(n)
    pair = torch.randn(n, n, 128, generator=g).bfloat16()
    if mask_dtype == torch.bool:
        mask = torch.rand(n, n, generator=g) > 0.3
    else:
        mask = torch.rand(n, n, generator=g).to(mask_dtype)
    mask[0, 1] = 0                       # asymmetric
    check_module(ref, hip, hnn.triangle_multiplication_hip, (pair.float(), mask.float()),
                 (pair.to(device), mask.to(device)), True, "trimul mask")


@pytest.mark.parametrize("n", [5, 37, 70])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_grid_self_attention(device, n, transpose, bf16):
    announce("grid_attention", n, transpose, bf16)
    ref, hip = pair_of("GridSelfAttention", dict(c_pair=128, num_head=4, transpose=transpose), seed=n)
    torch.manual_seed(n + 1)
    pair = torch.randn(n, n, 128)
    seq = torch.ones(n)
    seq[-3:] = 0
    mask = seq[:, None] * seq[None, :]
    mask[1, 2] = 0                       # asymmetric: the ending node must not transpose it
    if bf16:
        pair = pair.bfloat16()
    check_module(ref, hip, hnn.grid_self_attention_hip, (pair.float(), mask),
                 (pair.to(device), mask.to(device)), bf16, "grid attention")


@pytest.mark.parametrize("c,heads,n", [(64, 4, 40), (96, 4, 33), (128, 8, 70), (64, 2, 65), (48, 4, 37)])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_grid_self_attention_other_widths(device, c, heads, n, transpose, bf16):
    """Widths and head counts off the c = 128 / 4-head fast path: the template stack's 64
    channels in 4 heads of 16 (xfold/nn/template.py:192-195), 24-, 16-, 32- and 12-wide
    heads. In bf16 the attention runs in the pipelined kernel on operands repacked from the
    projections, in fp32 in the per-query kernel."""
    announce("grid_attention width", c, heads, n, transpose, bf16)
    ref, hip = pair_of("GridSelfAttention", dict(c_pair=c, num_head=heads, transpose=transpose), seed=c + n)
    torch.manual_seed(n + 3)
    pair = torch.randn(n, n, c)
    seq = torch.ones(n)
    seq[-3:] = 0
    mask = seq[:, None] * seq[None, :]
    mask[1, 2] = 0                       # asymmetric: the ending node must not transpose it
    if bf16:
        pair = pair.bfloat16()
    check_module(ref, hip, hnn.grid_self_attention_hip, (pair.float(), mask),
                 (pair.to(device), mask.to(device)), bf16, f"grid attention c={c} h={heads}")


def structured_pair_mask(n, seed):
    """Mask with every case the bf16 grid-attention kernel distinguishes per key block of 64:
    fully kept blocks, random holes, a row whose first block is fully masked, a row keeping
    one key, a column stripe masked for all rows, and fully masked (padding) rows."""
    g = torch.Generator().manual_seed(seed)
    mask = (torch.rand(n, n, generator=g) > 0.2).float()
    mask[8:24] = 1.0                     # row groups whose leading blocks are fully kept
    mask[3, :64] = 0.0                   # first key block fully masked for row 3
    mask[5] = 0.0
    mask[5, n - 12] = 1.0                # a single kept key, in the last (partial) block
    mask[:, 100:110] = 0.0               # a hole inside the second block, all rows
    mask[-10:] = 0.0                     # padding rows
    mask[:, -10:] = 0.0                  # padding keys
    return mask


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("sharp", [False, True])
def test_grid_self_attention_mask_cases(device, transpose, sharp):
    """bf16 fast path, n = 150 (three key blocks, the last partial). ``sharp`` scales the
    q/k projections by 2.5 and the bias projection by 4, so that logits span tens of units
    and the running maximum moves by more than the kernel's rescale slack between blocks;
    its bf16 rounding is then amplified (the bf16-operand floor's max error reaches ~0.13
    of the RMS), which the floor-relative max guard follows."""
    n = 150
    announce("grid_attention_masks", transpose, sharp)
    ref, hip = pair_of("GridSelfAttention", dict(c_pair=128, num_head=4, transpose=transpose), seed=7)
    if sharp:
        with torch.no_grad():
            for name, f in (("q_projection", 2.5), ("k_projection", 2.5), ("pair_bias_projection", 4.0)):
                getattr(ref, name).weight.mul_(f)
        hip.load_state_dict(ref.state_dict())
    torch.manual_seed(11)
    pair = torch.randn(n, n, 128).bfloat16()
    mask = structured_pair_mask(n, 5)
    got, want = run_both(ref, hip, (pair.float(), mask), (pair.to(device), mask.to(device)), True)
    floor = floor_of(lambda: ref(pair.float(), mask), stored=True)
    assert torch.isfinite(got.float()).all()
    assert_parity_bf16(got, want, "grid attention mask cases (bf16 store)", floor=floor)


@pytest.mark.parametrize("rows", [(37, 41), (300, 290)])
def test_transition_in_place(device, rows):
    """The pair stack's use: bf16 pair += transition(pair), in place."""
    announce("transition in place", rows)
    ref, hip = pair_of("Transition", dict(c_x=128, num_intermediate_factor=4), seed=7)
    torch.manual_seed(7)
    x = torch.randn(*rows, 128).bfloat16()
    with torch.no_grad():
        want = x.float() + ref(x.float())
    floor = bf16_stored(x.float() + floor_of(lambda: ref(x.float())))
    y = x.to(device)
    with torch.inference_mode(), autocast(True):
        hnn.transition_hip(hip, y, accumulate_into=y)
    assert_parity_bf16(y, want, "transition in place (bf16)", floor=floor)


@pytest.mark.parametrize("c,f,rows", [(128, 4, (33, 17)), (128, 4, (300, 290)), (384, 4, (50,)), (16, 4, (2, 5))])
@pytest.mark.parametrize("bf16", [False, True])
def test_transition(device, c, f, rows, bf16):
    announce("transition", c, f, rows, bf16)
    ref, hip = pair_of("Transition", dict(c_x=c, num_intermediate_factor=f), seed=c)
    x = torch.randn(*rows, c)
    if bf16:
        x = x.bfloat16()
    check_module(ref, hip, hnn.transition_hip, (x.float(),), (x.to(device),), bf16, "transition")


@pytest.mark.parametrize("cond", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
def test_self_attention(device, cond, bf16):
    c, heads, n = (768, 16, 40) if cond else (384, 16, 50)
    announce("self_attention", cond, bf16)
    ref, hip = pair_of("SelfAttention", dict(c_x=c, c_single_cond=384, num_head=heads, use_single_cond=cond),
                       seed=7)
    torch.manual_seed(8)
    x = torch.randn(2, n, c) if cond else torch.randn(n, c)
    mask = torch.ones(n)
    mask[-4:] = 0
    logits = torch.randn(heads, n, n)
    single = torch.randn(n, 384) if cond else None
    if bf16:
        x = x.bfloat16()
        logits = logits.bfloat16()
    dev = [t.to(device) if t is not None else None for t in (x, mask, logits, single)]
    check_module(ref, hip, hnn.self_attention_hip, (x.float(), mask, logits.float(), single), dev, bf16,
                 "self attention")


@pytest.mark.parametrize("c,heads,samples,n,mask_kind", [
    (768, 16, 5, 200, "tail"),          # the diffusion transformer's heads (Dh 48)
    (384, 16, 1, 77, "tail"),           # the Pairformer single track (Dh 24), ragged T
    (256, 4, 3, 130, "per_sample"),     # Dh 64, a different key mask per sample
    (128, 4, 2, 64, "none"),            # Dh 32, no mask
    (768, 16, 2, 40, "one_row_empty"),  # sample 1 keeps no key: uniform average of v
])
def test_self_attention_operand_path(device, monkeypatch, c, heads, samples, n, mask_kind):
    """bf16 SelfAttention with a packed bias: one GEMM writes q (pre-scaled), k, v^T and the
    gate straight into the attention kernel's layouts and the gate is applied at the
    attention's store. The general attention entry must not be called."""
    announce("self_attention operand path", c, heads, samples, n, mask_kind)
    monkeypatch.setattr(ops, "attention", lambda *a, **k: pytest.fail("general attention path taken"))
    ref, hip = pair_of("SelfAttention", dict(c_x=c, c_single_cond=64, num_head=heads, use_single_cond=True),
                       seed=c + n)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(samples, n, c, generator=g).bfloat16()
    logits = torch.randn(heads, n, n, generator=g)
    single = torch.randn(n, 64, generator=g)
    if mask_kind == "none":
        mask, rows = None, [None] * samples
    elif mask_kind == "tail":
        mask = torch.ones(n)
        mask[-5:] = 0
        rows = [mask] * samples
    else:
        mask = (torch.rand(samples, n, generator=g) > 0.3).float()
        mask[:, 0] = 1
        if mask_kind == "one_row_empty":
            mask[1] = 0
        rows = list(mask)

    def oracle():
        return torch.stack([ref(x[s].float(), rows[s], logits, single) for s in range(samples)])
    dev_mask = None if mask is None else mask.to(device)
    with torch.inference_mode():
        want = oracle()
        packed = ops.PackedBias(ops.attention_bias_pack(logits[None].to(device))[0])
        with autocast(True):
            got = hnn.self_attention_hip(hip, x.to(device), dev_mask, packed, single.to(device))
    assert_parity_bf16(got, want, "self attention operand path", floor=bf16_stored(floor_of(oracle)))


def test_attention_operands_reused(device):
    """One AttentionOperands set reused over calls with different inputs gives the same bits
    as a fresh set: the projection never writes the zero padding the kernel reads."""
    announce("attention operands reused")
    _, hip = pair_of("SelfAttention", dict(c_x=384, c_single_cond=64, num_head=16, use_single_cond=True), seed=3)
    hip = hip.to(device)
    g = torch.Generator().manual_seed(3)
    n = 70
    xs = [torch.randn(2, n, 384, generator=g).bfloat16().to(device) for _ in range(2)]
    mask = torch.ones(n, device=device)
    mask[-3:] = 0
    packed = ops.PackedBias(ops.attention_bias_pack(torch.randn(1, 16, n, n, generator=g).to(device))[0])
    single = torch.randn(n, 64, generator=g).to(device)
    shared = ops.AttentionOperands(2, n, 16, 24, device)
    with torch.inference_mode(), autocast(True):
        outs = [hnn.self_attention_hip(hip, x, mask, packed, single, _operands=shared) for x in xs]
        fresh = hnn.self_attention_hip(hip, xs[1], mask, packed, single)
    assert torch.equal(outs[1], fresh)
    assert not torch.equal(outs[0], outs[1])
    # The padding of q (head dims 24..31), k (keys >= 70) and v^T is still zero.
    q = shared.q.view(2, 16, n, shared.dp)
    assert q[..., 24:].abs().max().item() == 0
    k = shared.k.view(2, 16, shared.tpad, shared.dp)
    assert k[:, :, n:].abs().max().item() == 0 and k[..., 24:].abs().max().item() == 0
    vt = shared.vt.view(2, 16, shared.dp, shared.tpad)
    assert vt[:, :, 24:].abs().max().item() == 0


def test_attention_operand_mask_words_follow_the_mask(device):
    """The per-stream shared operand buffers recompute their kept-key words when the mask
    changes in place, when another mask tensor comes (even one allocated after the first is
    dropped) and for every inference-mode mask: each call equals one on fresh buffers."""
    announce("attention operand mask words")
    _, hip = pair_of("SelfAttention", dict(c_x=384, c_single_cond=64, num_head=16, use_single_cond=True), seed=4)
    g = torch.Generator().manual_seed(4)
    n = 96
    x = torch.randn(2, n, 384, generator=g).bfloat16().to(device)
    packed = ops.PackedBias(ops.attention_bias_pack(torch.randn(1, 16, n, n, generator=g).to(device))[0])
    single = torch.randn(n, 64, generator=g).to(device)

    def run(mask, fresh):
        operands = ops.AttentionOperands(2, n, 16, 24, device) if fresh else None
        with torch.no_grad(), autocast(True):
            return hnn.self_attention_hip(hip, x, mask, packed, single, _operands=operands)
    mask = torch.ones(n, device=device)
    mask[-5:] = 0
    first = run(mask, False)
    assert torch.equal(first, run(mask, True))
    mask[-30:] = 0                                    # in place: version bump
    second = run(mask, False)
    assert torch.equal(second, run(mask, True)) and not torch.equal(first, second)
    del mask
    other = torch.ones(n, device=device)
    other[:7] = 0
    third = run(other, False)
    assert torch.equal(third, run(other, True))
    with torch.inference_mode():
        inf_mask = torch.ones(n, device=device)
        inf_mask[10:20] = 0
    fourth = run(inf_mask, False)
    assert torch.equal(fourth, run(inf_mask, True)) and not torch.equal(third, fourth)


@pytest.mark.parametrize("B,T,H,Dh,K", [
    (2, 45, 4, 20, 64),   # V columns share tiles with k / gate: element stores
    (2, 48, 4, 16, 64),   # whole V tiles, T % 4 == 0: V^T from the swapped-operand MFMA
    (3, 64, 2, 32, 96),
])
def test_attention_project_layouts(device, B, T, H, Dh, K):
    """xfh_attention_project's layouts against the stacked projection computed by a plain
    GEMM: q = (x Wq^T + b) * qscale, k, v^T (keys permuted inside runs of 32) and the gate,
    at the bf16 bar (the layouts hold the bf16-rounded products)."""
    announce("attention project layouts", B, T, H, Dh, K)
    c = H * Dh
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B * T, K, generator=g).bfloat16().to(device)
    w = (torch.randn(4 * c, K, generator=g) / 8).bfloat16().to(device)
    bias = torch.randn(4 * c, generator=g).to(device)
    ops_ = ops.AttentionOperands(B, T, H, Dh, device)
    ops.attention_project(x, w, bias, ops_, 0.5)
    full = x.float() @ w.float().t() + bias                              # [B*T, 4c]
    parts = full.view(B, T, 4, H, Dh)
    q = ops_.q.view(B, H, T, ops_.dp)[..., :Dh].float()
    assert_parity(q, (parts[:, :, 0] * 0.5).permute(0, 2, 1, 3), TOL_BF16, "q layout")
    k = ops_.k.view(B, H, ops_.tpad, ops_.dp)[:, :, :T, :Dh].float()
    assert_parity(k, parts[:, :, 1].permute(0, 2, 1, 3), TOL_BF16, "k layout")
    pos = torch.tensor([(t & ~31) + ((t & 15) >> 2) * 8 + ((t & 31) >> 4) * 4 + (t & 3) for t in range(T)])
    vt = ops_.vt.view(B, H, ops_.dp, ops_.tpad)[:, :, :Dh].float()[..., pos.to(device)]
    assert_parity(vt, parts[:, :, 2].permute(0, 2, 3, 1), TOL_BF16, "v^T layout")
    assert_parity(ops_.gate.float(), parts[:, :, 3].reshape(B, T, c), TOL_BF16, "gate layout")
    # The padding stays zero: head-dim rows >= Dh, and the positions of keys >= T.
    vt_all = ops_.vt.view(B, H, ops_.dp, ops_.tpad)
    assert Dh == ops_.dp or vt_all[:, :, Dh:].abs().max().item() == 0
    pad_pos = [(t & ~31) + ((t & 15) >> 2) * 8 + ((t & 31) >> 4) * 4 + (t & 3) for t in range(T, ops_.tpad)]
    assert not pad_pos or vt_all[..., pad_pos].abs().max().item() == 0


@pytest.mark.parametrize("bf16", [False, True])
def test_diffusion_transition(device, bf16):
    announce("diffusion_transition", bf16)
    ref, hip = pair_of("DiffusionTransition", dict(c_x=768, c_single_cond=384, use_single_cond=True), seed=9)
    x, cond = torch.randn(2, 30, 768), torch.randn(30, 384)
    if bf16:
        x = x.bfloat16()
    check_module(ref, hip, hnn.diffusion_transition_hip, (x.float(), cond), (x.to(device), cond.to(device)),
                 bf16, "diffusion transition")


# ------------------------------------------------------------- gemm_ring configurations

def _ring_config(run):
    """Runs ``run`` with kernel timing on and returns the gemm_ring configuration it took
    (the library records each launch under "gemm_ring.<tile>[+xcd]")."""
    names = [f"gemm_ring.{t}{x}" for t in ("mid", "narrow", "shallow", "shallow_narrow", "xwide", "skinny")
             for x in ("", "+xcd")]
    for name in names:
        nh.kernel_timing_read(name)
    nh.set_kernel_timing(True)
    try:
        out = run()
        torch.cuda.synchronize()
    finally:
        nh.set_kernel_timing(False)
    taken = [name for name in names if nh.kernel_timing_read(name)[1]]
    return out, taken


@pytest.mark.parametrize("kind,m,k,n,batch,config", [
    ("linear", 3840, 768, 2304, 1, "xwide"),          # the diffusion QKV Linear
    ("glu", 3840, 768, 1536, 1, "xwide"),             # the diffusion transition's GLU
    ("linear", 2048, 768, 2304, 1, "mid"),
    ("linear", 3840, 768, 768, 1, "narrow+xcd"),      # per-XCD tile runs
    ("linear", 3840, 1536, 768, 1, "narrow+xcd"),
    ("linear", 512, 384, 128, 1, "narrow"),
    ("linear", 20000, 96, 256, 1, "shallow"),         # k % 64 != 0: 32-deep steps
    ("linear", 300, 96, 200, 1, "shallow_narrow"),
    ("batched", 768, 384, 768, 4, "narrow"),
    ("batched", 512, 768, 2304, 4, "mid"),
    ("linear", 150000, 64, 256, 1, "skinny+xcd"),     # k = 64 over many tiles (64-channel pairs)
    ("glu", 150000, 64, 128, 1, "skinny"),
])
def test_gemm_ring_configurations(device, kind, m, k, n, batch, config):
    """Every gemm_ring tile configuration, at shapes that select it on a 256-CU MI355X,
    against an fp32 matmul of the same bf16 operands."""
    announce("gemm_ring", kind, m, k, n, batch, config)
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    g = torch.Generator().manual_seed(m + k + n)
    x = torch.randn(batch, m, k, generator=g).bfloat16() if kind == "batched" else \
        torch.randn(m, k, generator=g).bfloat16()
    if kind == "glu":
        w = (torch.randn(2 * n, k, generator=g) / math.sqrt(k)).bfloat16()
        packed = nh._prepare(w.to(device), torch.bfloat16, "glu")
        got, taken = _ring_config(lambda: ops.gated_linear_unit(x.to(device), packed, n, torch.bfloat16))
        want = R.gated_linear_unit(x.float(), w.float().T)
    elif kind == "batched":
        w = (torch.randn(batch, n, k, generator=g) / math.sqrt(k)).bfloat16()
        bias = torch.randn(batch, n, generator=g)
        got, taken = _ring_config(lambda: ops.linear_batched(x.to(device), w.to(device), bias.to(device),
                                                             torch.bfloat16))
        want = torch.bmm(x.float(), w.float().transpose(1, 2).contiguous()) + bias[:, None, :]
    else:
        w = (torch.randn(n, k, generator=g) / math.sqrt(k)).bfloat16()
        bias = torch.randn(n, generator=g)
        got, taken = _ring_config(lambda: ops.linear(x.to(device), w.to(device), bias.to(device),
                                                     torch.bfloat16))
        want = x.float() @ w.float().T + bias
    assert taken == [f"gemm_ring.{config}"], taken
    # bf16 operands are exact in the fp32 reference: only accumulation order and the bf16
    # store differ, so the floor is the exact result stored in bf16.
    assert_parity_bf16(got, want, f"gemm_ring {config} {kind} {m}x{k}->{n}", floor=bf16_stored(want))


@pytest.mark.parametrize("profile", ["jump", "low", "ramp", "mixed"])
@pytest.mark.parametrize("batch", [3, 8])
def test_attention_logit_ranges(device, profile, batch):
    """The pipelined kernel's lazy running maximum (it rescales only when a row's maximum
    grows by more than a slack) across logit ranges (bias in natural units, fp32): 'jump'
    lifts the second half of the keys by 150, so every row rescales once mid-row; 'low'
    puts every logit near -300; 'ramp' raises the logits by up to 200 across the keys,
    block after block; 'mixed' gives each query its own offset in [-250, 250].
    Random key masks, 3 (a partial row group) or 8 batch rows, bf16 q/k/v."""
    announce("attention logit ranges", profile, batch)
    g = torch.Generator().manual_seed(batch)
    h, n, d = 4, 200, 32
    q, k, v = (torch.randn(batch, h, n, d, generator=g).bfloat16() for _ in range(3))
    bias = torch.randn(h, n, n, generator=g)
    if profile == "jump":
        bias[..., n // 2:] += 150.0
    elif profile == "low":
        bias -= 300.0
    elif profile == "ramp":
        bias += torch.linspace(-100.0, 200.0, n)
    else:
        bias += (torch.rand(1, n, 1, generator=g) - 0.5) * 500.0
    mask = torch.rand(batch, n, generator=g) > 0.2
    mask[:, 0] = True
    args = (q.float(), k.float(), v.float(), mask, bias)
    want = R.dot_product_attention(*args)
    floor = floor_of(lambda: R.dot_product_attention(*args), stored=True)
    got = ops.attention(q.to(device), k.to(device), v.to(device), mask.to(device), bias.to(device))
    assert torch.isfinite(got.float()).all()
    assert_parity_bf16(got, want, f"attention logits {profile}", floor=floor)
