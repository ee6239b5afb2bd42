"""Checkpoint records loaded straight into HBM (xfold_cpu_amd.params.load_params): the
device tensors equal the CPU reader's, sit in one device allocation, and a PairformerBlock
whose weights come from such a checkpoint matches the oracle block."""

import pytest
import torch

from oracle import restatement as R
from tests.helpers import TOL_FP32, assert_parity
from tests.test_gpu_ops import announce
from xfold_cpu_amd import nn as hnn
from xfold_cpu_amd.params import encode_record, load_params
from xfold_cpu_amd.synthetic import init_module_, pair_block_inputs

pytestmark = pytest.mark.gpu


def write_checkpoint(tmp_path, state, parts=3):
    blob = b"".join(encode_record("block", name, t) for name, t in state.items())
    cuts = [len(blob) * i // parts for i in range(parts + 1)]
    paths = []
    for i in range(parts):
        p = tmp_path / f"ckpt.part{i}"
        p.write_bytes(blob[cuts[i]:cuts[i + 1]])
        paths.append(p)
    return paths


@pytest.mark.parametrize("staging", [1 << 10, 1 << 20])
def test_device_load_matches_cpu_reader(device, tmp_path, staging):
    announce("load_params", staging)
    g = torch.Generator().manual_seed(0)
    state = {"w": torch.randn(300, 77, generator=g), "b": torch.randn(5, generator=g).bfloat16(),
             "h": torch.randn(3, 4, generator=g).half(), "u": torch.arange(13, dtype=torch.uint8),
             "s": torch.tensor(2.5), "e": torch.zeros(0, 4)}
    paths = write_checkpoint(tmp_path, state)
    cpu = load_params(paths)
    gpu = load_params(paths, device=device, staging_bytes=staging)
    assert sorted(cpu) == sorted(gpu) == sorted(f"block/{k}" for k in state)
    base = None
    for key, t in gpu.items():
        assert t.device.type == "cuda" and t.dtype == cpu[key].dtype and t.shape == cpu[key].shape
        torch.testing.assert_close(t.cpu(), cpu[key], rtol=0, atol=0)
        ptr = t.untyped_storage().data_ptr()
        base = base or ptr
        assert ptr == base                                  # one device allocation


def test_block_from_checkpoint(device, tmp_path):
    """fp32 PairformerBlock (N=40) with its weights read from a split checkpoint onto the GPU."""
    announce("block from checkpoint")
    args = dict(n_heads=4, c_pair=128, c_single=64, n_heads_pair=4)
    ref = init_module_(R.PairformerBlock(**args).eval(), seed=3, ln_jitter=True)
    paths = write_checkpoint(tmp_path, ref.state_dict())
    params = load_params(paths, device=device, staging_bytes=1 << 16)
    hip = hnn.PairformerBlock(**args).eval().to(device)
    hip.load_state_dict({k.split("/", 1)[1]: v for k, v in params.items()}, strict=True)
    inp = pair_block_inputs(40, c_pair=128, c_single=64, pad=2, seed=3)
    with torch.no_grad():
        want_pair, want_single = ref(inp.pair.clone(), inp.pair_mask, inp.single.clone(), inp.seq_mask)
    with torch.inference_mode():
        got_pair, got_single = hip(inp.pair.to(device), inp.pair_mask.to(device), inp.single.to(device),
                                   inp.seq_mask.to(device))
    assert_parity(got_pair, want_pair, TOL_FP32, "pair (checkpoint weights)")
    assert_parity(got_single, want_single, TOL_FP32, "single (checkpoint weights)")


def test_load_waits_for_work_queued_on_the_current_stream(device, tmp_path):
    """The device arena may be a block whose previous tensor is still to be read by work
    queued on the current stream; the upload's copies must start after that work."""
    announce("load_params after queued work")
    g = torch.Generator().manual_seed(5)
    state = {"w": torch.randn(1 << 18, generator=g)}           # 1 MiB: the arena's size
    paths = write_checkpoint(tmp_path, state, parts=1)
    cpu = load_params(paths)
    src = torch.randn(1 << 18, generator=g).to(device)         # a 1 MiB block of the same pool
    want = src.cpu() * 3
    torch.cuda.synchronize()
    torch.cuda._sleep(50_000_000)                              # holds the current stream
    out = src * 3                                              # reads src after the spin
    del src                                                    # its block is free for reuse
    gpu = load_params(paths, device=device, staging_bytes=1 << 16)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), want)
    assert torch.equal(gpu["block/w"].cpu(), cpu["block/w"])
