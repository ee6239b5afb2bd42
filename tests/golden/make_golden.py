"""Writes the golden fixtures in this directory from the reference's own modules.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py [/root/reference]

It imports the reference's ``xfold.nn`` modules (torch backend, CPU), initialises them
with ``xfold_cpu_amd.synthetic.init_module_`` (LayerNorm affine jittered), runs them on
seeded inputs in fp32 and under CPU bf16 autocast, and saves inputs, the state_dict and
outputs as ``.npz`` (data only). It covers the compositions that no closed form pins:
grid self-attention (both nodes), Transition, SelfAttention with and without
conditioning, DiffusionTransition, PairformerBlock, DiffusionTransformer,
EvoformerBlock (with OuterProductMean and MSAAttention inside) and the atom CrossAttention.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from xfold_cpu_amd.synthetic import init_module_, token_mask  # noqa: E402


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def save(name, module, args, inputs: dict, outputs: dict, meta: dict):
    payload = {"meta": np.array(json.dumps({"args": args, **meta}))}
    for k, v in inputs.items():
        if v is not None:
            payload[f"in/{k}"] = _np(v)
            payload[f"dtype/{k}"] = np.array(str(v.dtype))
    for k, v in module.state_dict().items():
        payload[f"param/{k}"] = _np(v)
    for k, v in outputs.items():
        payload[f"out/{k}"] = _np(v)
    np.savez_compressed(HERE / f"{name}.npz", **payload)
    print(f"wrote {name}.npz ({sum(a.size for a in payload.values())} values)")


def main(reference: str):
    sys.path.insert(0, reference)
    from xfold.fastnn import config
    from xfold.nn.attention import GridSelfAttention
    from xfold.nn.diffusion_transformer import CrossAttention, DiffusionTransformer, DiffusionTransition, SelfAttention
    from xfold.nn.pairformer import EvoformerBlock, PairformerBlock
    from xfold.nn.primitives import Transition

    for flag in ("layer_norm_implementation", "dot_product_attention_implementation",
                 "gated_linear_unit_implementation", "triangle_multiplication_implementation"):
        setattr(config, flag, "torch")
    config.input_cache_enabled = False
    torch.manual_seed(0)
    rng = np.random.RandomState(123)

    def randn(*shape):
        return torch.from_numpy(rng.standard_normal(shape).astype(np.float32))

    # Grid self-attention, starting and ending node, padded token + asymmetric mask.
    n, c, h = 7, 32, 4
    seq = token_mask(n, 1)
    pair_mask = seq[:, None] * seq[None, :]
    pair_mask[2, 4] = 0.0
    for transpose in (False, True):
        args = dict(c_pair=c, num_head=h, transpose=transpose)
        mod = init_module_(GridSelfAttention(**args).eval(), seed=1, ln_jitter=True)
        pair = randn(n, n, c)
        with torch.inference_mode():
            out = mod(pair, pair_mask)
        save(f"grid_attention_{'end' if transpose else 'start'}", mod, args,
             {"pair": pair, "mask": pair_mask}, {"out": out}, {"module": "GridSelfAttention"})

    # Transition (pair width, leading batch dims).
    args = dict(c_x=16, num_intermediate_factor=4)
    mod = init_module_(Transition(**args).eval(), seed=2, ln_jitter=True)
    x = randn(2, 5, 16)
    with torch.inference_mode():
        out = mod(x)
    save("transition", mod, args, {"x": x}, {"out": out}, {"module": "Transition"})

    # SelfAttention without conditioning (Pairformer single track) and with it (diffusion).
    n, c = 6, 32
    mask = token_mask(n, 1)
    logits = randn(4, n, n)
    args = dict(c_x=c, c_single_cond=16, num_head=4, use_single_cond=False)
    mod = init_module_(SelfAttention(**args).eval(), seed=3, ln_jitter=True)
    x = randn(n, c)
    with torch.inference_mode():
        out = mod(x, mask, pair_logits=logits)
    save("self_attention", mod, args, {"x": x, "mask": mask, "pair_logits": logits}, {"out": out},
         {"module": "SelfAttention"})
    args = dict(c_x=c, c_single_cond=16, num_head=4, use_single_cond=True)
    mod = init_module_(SelfAttention(**args).eval(), seed=4, ln_jitter=True)
    cond = randn(n, 16)
    with torch.inference_mode():
        out = mod(x, mask, pair_logits=logits, single_cond=cond)
    save("self_attention_cond", mod, args,
         {"x": x, "mask": mask, "pair_logits": logits, "single_cond": cond}, {"out": out},
         {"module": "SelfAttention"})

    # DiffusionTransition with conditioning.
    args = dict(c_x=32, c_single_cond=16, num_intermediate_factor=2, use_single_cond=True)
    mod = init_module_(DiffusionTransition(**args).eval(), seed=5, ln_jitter=True)
    with torch.inference_mode():
        out = mod(x, cond)
    save("diffusion_transition", mod, args, {"x": x, "single_cond": cond}, {"out": out},
         {"module": "DiffusionTransition"})

    # PairformerBlock, fp32 and CPU bf16 autocast (bf16 pair/single as in the full model).
    n = 6
    args = dict(n_heads=4, c_pair=32, c_single=24, n_heads_pair=4)
    mod = init_module_(PairformerBlock(**args).eval(), seed=6, ln_jitter=True)
    seq = token_mask(n, 1)
    pmask = seq[:, None] * seq[None, :]
    pair0, single0 = randn(n, n, 32), randn(n, 24)
    with torch.inference_mode():
        pair, single = mod(pair0.clone(), pmask, single0.clone(), seq)
    save("pairformer_block", mod, args,
         {"pair": pair0, "pair_mask": pmask, "single": single0, "seq_mask": seq},
         {"pair": pair, "single": single}, {"module": "PairformerBlock", "autocast": False})
    with torch.inference_mode(), torch.amp.autocast("cpu", dtype=torch.bfloat16):
        pair_b, single_b = mod(pair0.clone().bfloat16(), pmask, single0.clone().bfloat16(), seq)
    save("pairformer_block_bf16", mod, args,
         {"pair": pair0.bfloat16(), "pair_mask": pmask, "single": single0.bfloat16(), "seq_mask": seq},
         {"pair": pair_b, "single": single_b}, {"module": "PairformerBlock", "autocast": True})

    # DiffusionTransformer: 2 super-blocks of 2, 16 heads (the module's SelfAttention default).
    n = 5
    args = dict(c_act=64, c_single_cond=16, c_pair_cond=16, num_head=16, num_blocks=4, super_block_size=2)
    mod = init_module_(DiffusionTransformer(**args).eval(), seed=7, ln_jitter=True)
    act0, scond, pcond = randn(n, 64), randn(n, 16), randn(n, n, 16)
    dmask = token_mask(n, 1)
    with torch.inference_mode():
        out = mod(act0.clone(), dmask, scond, pcond)
    save("diffusion_transformer", mod, args,
         {"act": act0, "mask": dmask, "single_cond": scond, "pair_cond": pcond}, {"out": out},
         {"module": "DiffusionTransformer"})

    # EvoformerBlock (OuterProductMean, MSAAttention and the MSA transition before the pair
    # stack): the composition no closed form pins, with a partly masked MSA (a masked row,
    # scattered masked entries, one column masked in every row).
    n, s_rows = 6, 5
    args = dict(c_msa=16, c_pair=32, n_heads_pair=4)
    mod = init_module_(EvoformerBlock(**args).eval(), seed=8, ln_jitter=True)
    msa0, pair0 = randn(s_rows, n, 16), randn(n, n, 32)
    msa_mask = torch.from_numpy((rng.uniform(size=(s_rows, n)) > 0.25).astype(np.float32))
    msa_mask[2] = 0.0
    msa_mask[:, 4] = 0.0
    seq = token_mask(n, 1)
    pmask = seq[:, None] * seq[None, :]
    with torch.inference_mode():
        msa, pair = mod(msa0.clone(), pair0.clone(), msa_mask, pmask)
    save("evoformer_block", mod, args,
         {"msa": msa0, "pair": pair0, "msa_mask": msa_mask, "pair_mask": pmask},
         {"msa": msa, "pair": pair}, {"module": "EvoformerBlock"})

    # CrossAttention (atom queries over atom keys, per subset): a masked query, masked keys
    # (the positive 1e9 term then applies to the masked pairs) and pair logits.
    subsets, nq, nk, c = 3, 4, 6, 32
    args = dict(key_dim=c, value_dim=c, c_single_cond=c, num_head=4)
    mod = init_module_(CrossAttention(**args).eval(), seed=9, ln_jitter=True)
    x_q, x_k = randn(subsets, nq, c), randn(subsets, nk, c)
    mask_q = torch.ones(subsets, nq)
    mask_q[0, 3] = 0.0
    mask_k = torch.ones(subsets, nk)
    mask_k[0, 1] = 0.0
    mask_k[2, 5] = 0.0
    pair_logits = randn(subsets, 4, nq, nk)
    cond_q, cond_k = randn(subsets, nq, c), randn(subsets, nk, c)
    with torch.inference_mode():
        out = mod(x_q, x_k, mask_q, mask_k, pair_logits, cond_q, cond_k)
    save("cross_attention", mod, args,
         {"x_q": x_q, "x_k": x_k, "mask_q": mask_q, "mask_k": mask_k, "pair_logits": pair_logits,
          "single_cond_q": cond_q, "single_cond_k": cond_k},
         {"out": out}, {"module": "CrossAttention"})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
