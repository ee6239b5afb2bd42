"""Seeded synthetic weights and inputs for the benchmark configurations.

Weights: every ``nn.Linear`` weight ~ N(0, 1/fan_in), Linear biases ~ N(0, 1/fan_in),
LayerNorm gamma = 1 and beta = 0 (or, with ``ln_jitter``, gamma = 1 + 0.1 N(0,1) and
beta = 0.1 N(0,1) so that tests exercise the affine parameters), drawn in ``state_dict``
order from ``numpy.random.RandomState(seed)``. Activations come from a second stream,
``Generator(PCG64(seed + 1))`` (``activation_stream``). The same arrays can therefore be
loaded into the reference's modules, the CPU oracle and the HIP modules.

Configurations (the benchmark's ``configs``):
  C1  pair block, fp32, N=128, mask all ones
  C2  pair block, bf16, N=384, last 32 tokens padded
  C3  48-block trunk, bf16, N=768, single track, last ceil(0.1 N) = 77 tokens padded
  C4  diffusion transformer, 24 blocks, 5 samples, N=768, bf16, mask all ones
  C5  pair block, bf16, N=1536, 77 random tokens padded (5%)
"""

from __future__ import annotations

import concurrent.futures
import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch


def init_module_(module: torch.nn.Module, seed: int = 0, ln_jitter: bool = False) -> torch.nn.Module:
    rng = np.random.RandomState(seed)
    owners = dict(module.named_modules())
    params = dict(module.named_parameters())
    with torch.no_grad():
        for name in module.state_dict().keys():
            if name not in params:
                continue
            tensor = params[name]
            owner_name, _, pname = name.rpartition(".")
            owner = owners[owner_name]
            shape = tuple(tensor.shape)
            if type(owner).__name__ == "LayerNorm":
                if ln_jitter:
                    noise = rng.standard_normal(shape) * 0.1
                    value = 1.0 + noise if pname == "weight" else noise
                else:
                    value = np.ones(shape) if pname == "weight" else np.zeros(shape)
            elif tensor.dim() == 2:
                value = rng.standard_normal(shape) / math.sqrt(shape[1])
            elif tensor.dim() >= 3:
                # OuterProductMean.output_w [c, e, f]: fan-in c * e
                value = rng.standard_normal(shape) / math.sqrt(math.prod(shape[:-1]))
            else:
                w = getattr(owner, "weight", None)
                if w is None:                       # OuterProductMean.output_b
                    w = owner.output_w.reshape(-1, shape[0]).T
                value = rng.standard_normal(shape) / math.sqrt(w.shape[1])
            tensor.copy_(torch.from_numpy(np.asarray(value, dtype=np.float32)))
    return module


_PARTS = 16                  # independent sub-streams of one large draw (a fixed count)
_LARGE = 1 << 24


def normal(rng: np.random.Generator, shape) -> torch.Tensor:
    """N(0, 1) float32 of ``shape`` from ``rng``. Draws of more than 2^24 values are split
    along the first axis into 16 parts, each from its own stream spawned from ``rng``, and
    drawn on 16 threads: the result depends on the seed only, not on the thread count."""
    shape = tuple(shape)
    if math.prod(shape) <= _LARGE or shape[0] < _PARTS:
        return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32))
    out = np.empty(shape, dtype=np.float32)
    cuts = [shape[0] * i // _PARTS for i in range(_PARTS + 1)]
    streams = rng.spawn(_PARTS)

    def fill(i):
        streams[i].standard_normal(out=out[cuts[i]:cuts[i + 1]], dtype=np.float32)
    with concurrent.futures.ThreadPoolExecutor(max_workers=_PARTS) as pool:
        list(pool.map(fill, range(_PARTS)))
    return torch.from_numpy(out)


def activation_stream(seed: int) -> np.random.Generator:
    """The activations' generator: PCG64 with the ziggurat normal sampler (the N=1536 pair,
    302M values, in a few seconds, where the legacy RandomState takes ~45 s)."""
    return np.random.Generator(np.random.PCG64(seed + 1))


def token_mask(n: int, pad: int = 0, random_pad: bool = False, seed: int = 0) -> torch.Tensor:
    """1.0 for real tokens, 0.0 for padding (the last ``pad`` tokens, or ``pad`` random ones)."""
    m = np.ones(n, dtype=np.float32)
    if pad:
        if random_pad:
            m[np.random.RandomState(seed).choice(n, pad, replace=False)] = 0.0
        else:
            m[n - pad:] = 0.0
    return torch.from_numpy(m)


@dataclass
class PairBlockInputs:
    pair: torch.Tensor
    pair_mask: torch.Tensor
    single: Optional[torch.Tensor]
    seq_mask: torch.Tensor


def pair_block_inputs(n: int, c_pair: int = 128, c_single: int = 384, pad: int = 0,
                      random_pad: bool = False, seed: int = 0, with_single: bool = True) -> PairBlockInputs:
    rng = activation_stream(seed)
    pair = normal(rng, (n, n, c_pair))
    single = normal(rng, (n, c_single)) if with_single else None
    seq = token_mask(n, pad, random_pad, seed)
    return PairBlockInputs(pair, seq[:, None] * seq[None, :], single, seq)


@dataclass
class DiffusionInputs:
    act: torch.Tensor
    mask: torch.Tensor
    single_cond: torch.Tensor
    pair_cond: torch.Tensor


def diffusion_inputs(n: int, samples: int = 5, c_act: int = 768, c_single: int = 384,
                     c_pair: int = 128, seed: int = 0) -> DiffusionInputs:
    rng = activation_stream(seed)
    act = normal(rng, (samples, n, c_act))
    single_cond = normal(rng, (n, c_single))
    pair_cond = normal(rng, (n, n, c_pair))
    return DiffusionInputs(act, torch.ones(n), single_cond, pair_cond)


CONFIGS = {
    "C1": dict(kind="pair_block", n=128, dtype="fp32", pad=0, random_pad=False, with_single=False),
    "C2": dict(kind="pair_block", n=384, dtype="bf16", pad=32, random_pad=False, with_single=False),
    "C3": dict(kind="trunk", n=768, dtype="bf16", pad=77, random_pad=False, with_single=True, blocks=48),
    "C4": dict(kind="diffusion", n=768, dtype="bf16", samples=5, blocks=24),
    "C5": dict(kind="pair_block", n=1536, dtype="bf16", pad=77, random_pad=True, with_single=False),
    # The template stack's block (xfold/nn/template.py:192-195): 64 pair channels, 4 heads of
    # 16, transition factor 2; not a BASELINE configuration (bench.py --config T768).
    "T768": dict(kind="pair_block", n=768, dtype="bf16", pad=77, random_pad=False, with_single=False,
                 c_pair=64, factor=2),
}
