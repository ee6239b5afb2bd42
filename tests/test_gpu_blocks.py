"""Per-block parity (PairformerBlock, DiffusionTransformer) and the golden fixtures
through the HIP modules."""

import pytest
import torch

from oracle import restatement as R
from tests.helpers import (TOL_BF16, TOL_FP32, assert_parity, assert_parity_bf16, floor_of,
                           load_fixture, rel_err, residual)
from tests.test_gpu_ops import announce, autocast, pair_of
from xfold_cpu_amd import nn as hnn
from xfold_cpu_amd.synthetic import init_module_, pair_block_inputs

pytestmark = pytest.mark.gpu


def run_hip_fixture(name, device):
    meta, inputs, params, outputs = load_fixture(name)
    module = getattr(hnn, meta["module"])(**meta["args"]).eval()
    module.load_state_dict(params, strict=True)
    module.to(device)
    d = {k: v.to(device) for k, v in inputs.items()}
    bf16 = meta.get("autocast", False)
    kind = meta["module"]
    with torch.inference_mode(), autocast(bf16):
        if kind == "GridSelfAttention":
            got = {"out": module(d["pair"], d["mask"])}
        elif kind == "Transition":
            got = {"out": module(d["x"])}
        elif kind == "SelfAttention":
            got = {"out": module(d["x"], d["mask"], d["pair_logits"], d.get("single_cond"))}
        elif kind == "DiffusionTransition":
            got = {"out": module(d["x"], d["single_cond"])}
        elif kind == "PairformerBlock":
            pair, single = module(d["pair"].clone(), d["pair_mask"], d["single"].clone(), d["seq_mask"])
            got = {"pair": pair, "single": single}
        elif kind == "CrossAttention":
            got = {"out": module(d["x_q"], d["x_k"], d["mask_q"], d["mask_k"], d["pair_logits"],
                                 d["single_cond_q"], d["single_cond_k"])}
        else:
            got = {"out": module(d["act"].clone(), d["mask"], d["single_cond"], d["pair_cond"])}
    return meta, got, outputs


@pytest.mark.parametrize("name", ["grid_attention_start", "grid_attention_end", "transition",
                                  "self_attention", "self_attention_cond", "diffusion_transition",
                                  "pairformer_block", "diffusion_transformer", "cross_attention"])
def test_golden_vectors_through_hip(device, name):
    """fp32 golden vectors written by the reference's own modules."""
    announce("golden", name)
    meta, got, want = run_hip_fixture(name, device)
    for key in want:
        assert_parity(got[key], want[key], TOL_FP32, f"{name}/{key}")


def test_golden_bf16_pairformer_block(device):
    """The reference's own bf16 block (CPU autocast, golden fixture): both it and the HIP
    bf16 block are measured against the fp32 oracle on the fixture's bf16 inputs."""
    meta, got, ref_bf16 = run_hip_fixture("pairformer_block_bf16", device)
    _, inputs, params, _ = load_fixture("pairformer_block_bf16")
    ref = R.PairformerBlock(**meta["args"]).eval()
    ref.load_state_dict(params)
    def oracle(wrap=lambda t: t):
        return ref(wrap(inputs["pair"].float().clone()), inputs["pair_mask"],
                   wrap(inputs["single"].float().clone()), inputs["seq_mask"])
    with torch.inference_mode():
        exact_pair, exact_single = oracle()
    # The HIP block keeps the fixture's bf16 pair and single: a bf16 residual stream.
    floor_pair, floor_single = floor_of(lambda: oracle(residual))
    for key, exact, floor in (("pair", exact_pair, floor_pair), ("single", exact_single, floor_single)):
        print(f"[bf16 block/{key}] reference-bf16 max {rel_err(ref_bf16[key], exact):.3e}")
        assert_parity_bf16(got[key], exact, f"golden bf16 block/{key}", floor=floor)


def block_case(n, c_single, mode, pad, seed, device, with_single=True, c_pair=128, factor=4):
    """mode: 'fp32' (fp32 pair, no autocast), 'bf16-compute' (fp32 pair, bf16 autocast),
    'bf16' (bf16 pair and single under bf16 autocast, the C2-C5 protocol)."""
    args = dict(n_heads=16, c_pair=c_pair, c_single=c_single, n_heads_pair=4, with_single=with_single,
                num_intermediate_factor=factor)
    ref, hip = pair_of("PairformerBlock", args, seed=seed, device=device)
    inp = pair_block_inputs(n, c_pair=c_pair, c_single=c_single, pad=pad, seed=seed, with_single=with_single)
    pair, single = inp.pair, inp.single
    if mode == "bf16":
        pair = pair.bfloat16()
        single = single.bfloat16() if single is not None else None
    def oracle(wrap=lambda t: t):
        if with_single:
            return ref(wrap(pair.float().clone()), inp.pair_mask, wrap(single.float().clone()), inp.seq_mask)
        return ref(wrap(pair.float().clone()), inp.pair_mask), None
    floor_pair = floor_single = None
    if mode == "bf16":                  # bf16 residual stream
        floor_pair, floor_single = floor_of(lambda: oracle(residual))
    elif mode == "bf16-compute":
        floor_pair, floor_single = floor_of(oracle)
    with torch.inference_mode():
        want_pair, want_single = oracle()
        dp = pair.to(device).contiguous()
        ds = single.to(device).contiguous() if single is not None else None
        with autocast(mode != "fp32"):
            if with_single:
                got_pair, got_single = hip(dp, inp.pair_mask.to(device), ds, inp.seq_mask.to(device))
            else:
                got_pair, got_single = hip(dp, inp.pair_mask.to(device)), None
    return (got_pair, want_pair, floor_pair), (got_single, want_single, floor_single)


@pytest.mark.parametrize("n,mode", [(24, "fp32"), (48, "bf16-compute"), (96, "bf16-compute"),
                                    (48, "bf16"), (96, "bf16"), (200, "bf16")])
def test_pairformer_block(device, n, mode):
    announce("pairformer_block", n, mode)
    (gp, wp, fp), (gs, ws, fs) = block_case(n, 384, mode, pad=3, seed=n, device=device)
    if mode == "fp32":
        assert gp.dtype == torch.float32
        assert_parity(gp, wp, TOL_FP32, "pair")
        assert_parity(gs, ws, TOL_FP32, "single")
    elif mode == "bf16-compute":
        assert gp.dtype == torch.float32
        assert_parity_bf16(gp, wp, "pair", floor=fp)
        assert_parity_bf16(gs, ws, "single", floor=fs)
    else:
        # The residual stream is bf16, as in the reference's full model under autocast: pair
        # is rounded at each of its 5 in-place updates, single at its 2 (and so is the floor).
        assert gp.dtype == torch.bfloat16
        assert_parity_bf16(gp, wp, "pair", floor=fp)
        assert_parity_bf16(gs, ws, "single", floor=fs)


@pytest.mark.parametrize("n,mode,pad", [(1, "fp32", 0), (1, "bf16", 0), (2, "bf16", 1), (3, "fp32", 0),
                                        (3, "bf16", 3)])
def test_pairformer_block_tiny(device, n, mode, pad):
    """One to three tokens (one token padded, or all of them): every kernel's tail and
    padding logic at its smallest, fully masked rows included."""
    announce("pairformer_block tiny", n, mode, pad)
    (gp, wp, fp), (gs, ws, fs) = block_case(n, 64, mode, pad=pad, seed=n + 3, device=device)
    assert torch.isfinite(gp.float()).all() and torch.isfinite(gs.float()).all()
    if mode == "fp32":
        assert_parity(gp, wp, TOL_FP32, "pair")
        assert_parity(gs, ws, TOL_FP32, "single")
    else:
        assert_parity_bf16(gp, wp, "pair", floor=fp)
        assert_parity_bf16(gs, ws, "single", floor=fs)


@pytest.mark.parametrize("n,mode", [(40, "fp32"), (40, "bf16"), (150, "bf16")])
def test_template_pairformer_block(device, n, mode):
    """The template stack's block (xfold/nn/template.py:192-195): c_pair 64, transition
    factor 2, 4 pair heads of 16 channels, no single track."""
    announce("template_block", n, mode)
    (gp, wp, fp), _ = block_case(n, 0, mode, pad=2, seed=n + 7, device=device, with_single=False,
                                 c_pair=64, factor=2)
    if mode == "fp32":
        assert_parity(gp, wp, TOL_FP32, "pair")
    else:
        assert gp.dtype == torch.bfloat16
        assert_parity_bf16(gp, wp, "pair", floor=fp)


def test_pairformer_block_updates_in_place(device):
    args = dict(n_heads=4, c_pair=128, c_single=64, n_heads_pair=4)
    _, hip = pair_of("PairformerBlock", args, seed=1, device=device)
    inp = pair_block_inputs(16, c_single=64, seed=1)
    pair, single = inp.pair.to(device), inp.single.to(device)
    with torch.inference_mode():
        p2, s2 = hip(pair, inp.pair_mask.to(device), single, inp.seq_mask.to(device))
    assert p2.data_ptr() == pair.data_ptr() and s2.data_ptr() == single.data_ptr()


def test_pairformer_block_fused_transition_logits(device, monkeypatch):
    """The block with its pair transition and pair logits in one kernel gives the same pair
    and single, bit for bit, as with the two kernels."""
    from xfold_cpu_amd.nn import pairformer as P
    announce("pairformer_block fused transition+logits", 72)
    args = dict(n_heads=16, c_pair=128, c_single=384, n_heads_pair=4)
    _, hip = pair_of("PairformerBlock", args, seed=5, device=device)
    inp = pair_block_inputs(72, pad=5, seed=5)
    outs = []
    for fused in (True, False):
        monkeypatch.setattr(P, "FUSE_TRANSITION_AND_LOGITS", fused)
        pair, single = inp.pair.bfloat16().to(device), inp.single.bfloat16().to(device)
        with torch.inference_mode(), torch.amp.autocast("cuda", dtype=torch.bfloat16):
            outs.append(hip(pair, inp.pair_mask.to(device), single, inp.seq_mask.to(device)))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("mode", ["fp32", "bf16-compute", "bf16"])
def test_diffusion_transformer_batched_samples(device, mode):
    """Five samples batched in one call equal the reference's one-sample-at-a-time loop."""
    announce("diffusion_transformer", mode)
    bf16 = mode != "fp32"
    args = dict(c_act=256, c_single_cond=64, c_pair_cond=32, num_head=16, num_blocks=4, super_block_size=2)
    ref, hip = pair_of("DiffusionTransformer", args, seed=11, device=device)
    torch.manual_seed(11)
    n, samples = 33, 5
    act = torch.randn(samples, n, 256)
    mask = torch.ones(n)
    mask[-2:] = 0
    scond, pcond = torch.randn(n, 64), torch.randn(n, n, 32)
    if mode == "bf16":
        act = act.bfloat16()
    def oracle(wrap=lambda t: t):
        return torch.stack([ref(wrap(act[s].float().clone()), mask, scond, pcond) for s in range(samples)])
    with torch.inference_mode():
        want = oracle()
        with autocast(bf16):
            got = hip(act.to(device).clone(), mask.to(device), scond.to(device), pcond.to(device))
    if not bf16:
        assert_parity(got, want, TOL_FP32, "diffusion transformer")
        return
    # In "bf16" mode act is a bf16 residual stream rounded at each of its 2 updates per block.
    floor = floor_of(lambda: oracle(residual if mode == "bf16" else (lambda t: t)))
    assert_parity_bf16(got, want, "diffusion transformer", floor=floor)


def test_unpacked_bias_beyond_the_attention_key_limit(device, monkeypatch):
    """Token counts above the pipelined attention kernel's key limit take the unpacked
    [H, N, N] bias path (the general attention kernel) in the block's single track and in
    the diffusion transformer: with the limit lowered to 32, N = 40 must still match the
    oracle."""
    from xfold_cpu_amd.fastnn import native_hip as nh
    monkeypatch.setattr(nh, "attention_max_keys", lambda: 32)
    (gp, wp, fp), (gs, ws, fs) = block_case(40, 64, "bf16", pad=3, seed=5, device=device)
    assert_parity_bf16(gp, wp, "pair (limit 32)", floor=fp)
    assert_parity_bf16(gs, ws, "single (limit 32)", floor=fs)
    args = dict(c_act=256, c_single_cond=64, c_pair_cond=128, num_head=16, num_blocks=2, super_block_size=2)
    ref, hip = pair_of("DiffusionTransformer", args, seed=6, device=device)
    g = torch.Generator().manual_seed(6)
    n = 40
    act = torch.randn(2, n, 256, generator=g).bfloat16()
    mask = torch.ones(n)
    mask[-3:] = 0
    scond, pcond = torch.randn(n, 64, generator=g), torch.randn(n, n, 128, generator=g)

    def oracle(wrap=lambda t: t):
        return torch.stack([ref(wrap(act[s].float().clone()), mask, scond, pcond) for s in range(2)])
    with torch.inference_mode():
        want = oracle()
        with autocast(True):
            got = hip(act.to(device).clone(), mask.to(device), scond.to(device), pcond.to(device))
    assert_parity_bf16(got, want, "diffusion transformer (limit 32)", floor=floor_of(lambda: oracle(residual)))


def test_diffusion_input_cache_skips_the_pair_logits_on_repeat_calls(device):
    """Inside an input-cache scope (the reference's InputCache rules) a second call with the
    same pair_cond and weights reuses the packed pair logits (no pair_bias_kernel launch)
    and gives the same result bit for bit; an in-place update of pair_cond invalidates them."""
    from xfold_cpu_amd.fastnn import config
    from xfold_cpu_amd.fastnn import native_hip as nh
    from xfold_cpu_amd.nn.cache import input_cache_scope
    args = dict(c_act=256, c_single_cond=64, c_pair_cond=128, num_head=16, num_blocks=4, super_block_size=2)
    _, hip = pair_of("DiffusionTransformer", args, seed=8, device=device)
    g = torch.Generator().manual_seed(8)
    n = 50
    act = torch.randn(3, n, 256, generator=g).bfloat16().to(device)
    mask = torch.ones(n, device=device)
    scond, pcond = torch.randn(n, 64, generator=g).to(device), torch.randn(n, n, 128, generator=g).to(device)

    def run():
        nh.kernel_timing_read("pair_bias")
        nh.set_kernel_timing(True)
        try:
            with torch.inference_mode(), autocast(True):
                out = hip(act.clone(), mask, scond, pcond)
            torch.cuda.synchronize()
        finally:
            nh.set_kernel_timing(False)
        return out, nh.kernel_timing_read("pair_bias")[1]
    saved = config.input_cache_enabled
    config.input_cache_enabled = True
    try:
        with torch.no_grad(), input_cache_scope():
            first, launches1 = run()
            second, launches2 = run()
            pcond.add_(0.5)
            third, launches3 = run()
        uncached, launches4 = run()                     # outside the scope: recomputed
    finally:
        config.input_cache_enabled = saved
    assert (launches1, launches2, launches3, launches4) == (1, 0, 1, 1)
    assert torch.equal(first, second)
    assert torch.equal(third, uncached)
    assert not torch.equal(first, third)


def test_glu_reuses_its_packed_weight_with_a_foreign_cache(device):
    """gated_linear_unit(x, weight, weight_cache) with a cache object of the reference's
    kind (not a HipWeightCache) packs the weight once per weight version."""
    import importlib
    from xfold_cpu_amd import fastnn
    glu_mod = importlib.import_module("xfold_cpu_amd.fastnn.gated_linear_unit")

    class GLUWeightCache:                 # a stand-in with the reference's name and no methods used
        pass
    cache = GLUWeightCache()
    lin = torch.nn.Linear(128, 2 * 256, bias=False).to(device)
    x = torch.randn(40, 128, device=device)
    with torch.inference_mode(), autocast(True):
        a = fastnn.gated_linear_unit(x, lin.weight.T, weight_cache=cache)
        packed = glu_mod._attached[cache]._value
        b = fastnn.gated_linear_unit(x, lin.weight.T, weight_cache=cache)
        assert glu_mod._attached[cache]._value is packed
    assert torch.equal(a, b)
    with torch.no_grad():
        lin.weight.mul_(2)
    with torch.inference_mode(), autocast(True):
        fastnn.gated_linear_unit(x, lin.weight.T, weight_cache=cache)
        assert glu_mod._attached[cache]._value is not packed
