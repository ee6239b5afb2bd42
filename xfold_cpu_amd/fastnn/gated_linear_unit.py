"""``gated_linear_unit(x, weight, weight_cache=None)`` with the reference's signature
(``xfold/fastnn/gated_linear_unit.py:110-122``): ``weight`` is ``[K, 2F]`` (callers pass
``transition1.weight.T``), the first F columns are the SiLU gate."""

from __future__ import annotations

import weakref

import torch

from . import config as fastnn_config
from . import native_hip as nh
from . import ops

# Device caches attached to caller-owned cache objects that are not HipWeightCaches (the
# reference's GLUWeightCache, xfold/fastnn/gated_linear_unit.py:6-48, which Transition
# passes on every call): one packed copy per such object, released with it.
_attached = weakref.WeakKeyDictionary()


def _device_cache(weight_cache):
    if weight_cache is None or isinstance(weight_cache, nh.HipWeightCache):
        return weight_cache
    try:
        cache = _attached.get(weight_cache)
        if cache is None:
            cache = _attached[weight_cache] = nh.HipWeightCache()
        return cache
    except TypeError:                 # not weak-referenceable: no reuse across calls
        return None


def gated_linear_unit_hip(x: torch.Tensor, weight: torch.Tensor, weight_cache=None) -> torch.Tensor:
    nh.check_gpu_inference(x, weight)
    dtype = nh.compute_dtype(x, weight)
    if weight.dim() != 2 or weight.shape[1] % 2 or weight.shape[0] != x.shape[-1]:
        raise ValueError("gated_linear_unit: weight must be [K, 2F] matching x's last dim")
    f = weight.shape[1] // 2
    # The cache holds the packed copy of weight.T ([2F, K], nn.Linear layout), keyed on the
    # weight's version like the reference's GLUWeightCache.
    cache = _device_cache(weight_cache)
    source = weight.T
    packed = cache.get(source, dtype, "glu") if cache is not None else nh._prepare(source, dtype, "glu")
    return ops.gated_linear_unit(x, packed, f, dtype)


def gated_linear_unit(x: torch.Tensor, weight: torch.Tensor, weight_cache=None) -> torch.Tensor:
    if fastnn_config.gated_linear_unit_implementation == fastnn_config.HIP:
        return gated_linear_unit_hip(x, weight, weight_cache)
    raise ValueError("Unknown gated_linear_unit_implementation for xfold_cpu_amd: "
                     f"{fastnn_config.gated_linear_unit_implementation!r} (only 'hip')")
