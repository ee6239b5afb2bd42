"""HIP-graph capture of the HIP modules (torch.cuda.CUDAGraph): a bf16 PairformerBlock
(xfold/nn/pairformer.py:77-114) and a DiffusionTransformer forward
(xfold/nn/diffusion_transformer.py:250-272) are captured once and replayed several times, with
eager work and synchronisations between the replays; every replay must equal the eager
result bit for bit (the kernels are deterministic and the path records no memset, host copy
or synchronisation). The replayed Pairformer block is also held to the fp32 CPU oracle
(oracle/restatement.py) and its bf16 floor, the bar of the eager tests."""

import pytest
import torch

from tests.helpers import assert_parity_bf16, floor_of, residual
from tests.test_gpu_ops import announce, autocast, pair_of
from xfold_cpu_amd.synthetic import pair_block_inputs

pytestmark = pytest.mark.gpu


def capture(fn):
    """Warm up on a side stream (weight caches are built outside the capture), then capture."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def replay_and_check(graph, reset, outputs, wants, replays=3, check=None):
    """Replays `graph` after `reset()`; every replay's outputs must equal `wants` bit for bit
    and pass `check(outputs)` when one is given."""
    for rep in range(replays):
        reset()
        graph.replay()
        torch.cuda.synchronize()
        # Eager work on the same stream between replays.
        scratch = torch.randn(1 << 16, device=outputs[0].device).sum()
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        for got, want in zip(outputs, wants):
            assert torch.equal(got, want), f"replay {rep} differs from the eager result"
        if check is not None:
            check(outputs)


@pytest.mark.parametrize("n", [48, 100])
def test_pairformer_block_graph_replay(device, n):
    announce("graph pairformer_block", n)
    args = dict(n_heads=16, c_pair=128, c_single=384, n_heads_pair=4)
    ref, hip = pair_of("PairformerBlock", args, seed=n, device=device)
    inp = pair_block_inputs(n, pad=3, seed=n)
    pair0, single0 = inp.pair.bfloat16().to(device), inp.single.bfloat16().to(device)
    pm, sm = inp.pair_mask.to(device), inp.seq_mask.to(device)
    pair, single = pair0.clone(), single0.clone()

    def oracle(wrap=lambda t: t):
        return ref(wrap(inp.pair.bfloat16().float()), inp.pair_mask, wrap(inp.single.bfloat16().float()),
                   inp.seq_mask)
    with torch.inference_mode():
        want_pair_ref, want_single_ref = oracle()
    floor_pair, floor_single = floor_of(lambda: oracle(residual))

    def against_oracle(outputs):
        got_pair, got_single = outputs
        assert_parity_bf16(got_pair, want_pair_ref, f"graph replay PairformerBlock N={n} pair", floor=floor_pair)
        assert_parity_bf16(got_single, want_single_ref, f"graph replay PairformerBlock N={n} single",
                           floor=floor_single)

    def reset():
        pair.copy_(pair0)
        single.copy_(single0)

    def block():
        hip(pair, pm, single, sm)

    with torch.inference_mode(), autocast(True):
        block()                                    # eager result
        torch.cuda.synchronize()
        want_pair, want_single = pair.clone(), single.clone()
        reset()
        graph = capture(block)
        replay_and_check(graph, reset, (pair, single), (want_pair, want_single), check=against_oracle)


def test_diffusion_transformer_graph_replay(device):
    announce("graph diffusion_transformer")
    args = dict(c_act=256, c_single_cond=64, c_pair_cond=128, num_head=16, num_blocks=4, super_block_size=2)
    _, hip = pair_of("DiffusionTransformer", args, seed=5, device=device)
    torch.manual_seed(5)
    n, samples = 40, 3
    act0 = torch.randn(samples, n, 256).bfloat16().to(device)
    mask = torch.ones(n)
    mask[-3:] = 0
    mask = mask.to(device)
    scond, pcond = torch.randn(n, 64).to(device), torch.randn(n, n, 128).to(device)
    act = act0.clone()
    out = {}

    def reset():
        act.copy_(act0)

    def forward():
        out["act"] = hip(act, mask, scond, pcond)

    with torch.inference_mode(), autocast(True):
        forward()
        torch.cuda.synchronize()
        want = out["act"].clone()
        reset()
        graph = capture(forward)
        replay_and_check(graph, reset, (out["act"],), (want,))
