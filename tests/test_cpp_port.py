"""The CPU baseline's restatement of the reference's cpp backend (oracle/cpp_port.py,
oracle/cpp/af3_port.cpp) against the torch restatement: the same results in fp32 (1e-4
of the RMS; only tile GEMM order differs) and at the bf16 bar under CPU bf16 autocast,
per operator and per block. Skipped when the extension has not been built
(``__graft_entry__.build()`` builds it)."""

import pytest
import torch

from oracle import restatement as R
from tests.helpers import TOL_FP32, assert_parity, rms_rel_err
from xfold_cpu_amd.synthetic import init_module_, pair_block_inputs

cpp_port = pytest.importorskip("oracle.cpp_port")
try:
    cpp_port.load()
except RuntimeError as err:                      # not built in this checkout
    pytest.skip(str(err), allow_module_level=True)


def test_tiled_matmul_and_glu_match_matmul():
    g = torch.Generator().manual_seed(0)
    x, w, b = torch.randn(300, 96, generator=g), torch.randn(96, 260, generator=g), torch.randn(260, generator=g)
    assert_parity(cpp_port.load().tiled_matmul(x, w, b), x @ w + b, TOL_FP32, "tiled_matmul")
    a3, b3 = torch.randn(3, 130, 40, generator=g), torch.randn(3, 40, 129, generator=g)
    assert_parity(cpp_port.load().tiled_matmul(a3, b3, None), torch.bmm(a3, b3), TOL_FP32, "batched")
    wg = torch.randn(96, 2 * 150, generator=g)
    assert_parity(cpp_port.gated_linear_unit_cpp(x, wg), R.gated_linear_unit(x, wg), TOL_FP32, "glu")


@pytest.mark.parametrize("mask_rank", [None, 1, 2])
def test_attention_matches_restatement(mask_rank):
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(2, 3, 150, 16, generator=g) for _ in range(3))
    bias = torch.randn(3, 150, 150, generator=g)
    keep = torch.rand(2, 150, generator=g) > 0.3
    keep[1] = False                                   # fully masked row: uniform over all keys
    mask = None if mask_rank is None else keep[0] if mask_rank == 1 else keep
    want = R.dot_product_attention(q, k, v, mask, bias)
    assert_parity(cpp_port.dot_product_attention_cpp(q, k, v, mask, bias), want, TOL_FP32, "attention")


@pytest.mark.parametrize("with_single", [False, True])
def test_pairformer_block_fp32_and_bf16(with_single):
    n = 40
    block = init_module_(R.PairformerBlock(n_heads=16, c_single=64, with_single=with_single).eval(),
                         seed=3, ln_jitter=True)
    inp = pair_block_inputs(n, c_single=64, pad=4, seed=3, with_single=with_single)
    cpp = cpp_port.PairformerBlockCpp(block)
    with torch.inference_mode():
        args = (inp.pair_mask,) if not with_single else (inp.pair_mask, None, inp.seq_mask)
        for bf16 in (False, True):
            pair = inp.pair.clone()
            single = inp.single.clone() if with_single else None
            want = block(pair.clone(), inp.pair_mask, None if single is None else single.clone(), inp.seq_mask)
            with torch.amp.autocast("cpu", dtype=torch.bfloat16, enabled=bf16):
                got = cpp(pair.clone(), inp.pair_mask, None if single is None else single.clone(), inp.seq_mask)
            want = want if with_single else (want,)
            got = got if with_single else (got,)
            for gt, wt in zip(got, want):
                if bf16:
                    assert rms_rel_err(gt.float(), wt) < 2e-2
                else:
                    assert_parity(gt, wt, TOL_FP32, "cpp block")


def test_diffusion_transformer_fp32():
    args = dict(c_act=128, c_single_cond=32, c_pair_cond=16, num_head=16, num_blocks=2, super_block_size=2)
    m = init_module_(R.DiffusionTransformer(**args).eval(), seed=5, ln_jitter=True)
    g = torch.Generator().manual_seed(5)
    n = 20
    act, scond, pcond = torch.randn(n, 128, generator=g), torch.randn(n, 32, generator=g), torch.randn(n, n, 16, generator=g)
    mask = torch.ones(n)
    mask[-2:] = 0
    with torch.inference_mode():
        want = m(act.clone(), mask, scond, pcond)
        got = cpp_port.DiffusionTransformerCpp(m)(act.clone(), mask, scond, pcond)
    assert_parity(got, want, TOL_FP32, "cpp diffusion transformer")
