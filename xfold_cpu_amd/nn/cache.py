"""Example-scoped input cache with the reference's interface and invalidation rules
(``xfold/nn/cache.py:1-151``), for the hip DiffusionTransformer's static per-example inputs
(the packed pair logits of every super-block and every block's conditioning).

Semantics kept from the reference, because a caller switching backends must see the same
reuse and invalidation:
  * entries live only inside ``input_cache_scope()`` while ``config.input_cache_enabled`` is
    set, the owner and the listed modules are in eval mode and grad mode is off; leaving the
    scope (normally or by an exception) releases them (``cache.py:84-95, 114-116``);
  * the key covers the scope, every dependency (tensor identity, address, version counter,
    shape, strides, dtype, device; versionless inference tensors only as dependencies), the
    listed modules' parameters (never versionless ones), their ``eps``/``normalized_shape``,
    the CUDA and CPU autocast state and the backend switches (``cache.py:19-41, 120-130``);
  * all caches of one scope share ``config.input_cache_max_bytes``; an entry that does not
    fit is returned uncached (``cache.py:73-82, 140-146``).
"""

from __future__ import annotations

import dataclasses
from contextlib import contextmanager
from contextvars import ContextVar

import torch

from ..fastnn import config

_SCOPE = ContextVar("xfold_cpu_amd_input_cache_scope", default=None)


class _NotCacheable(Exception):
    pass


def _tensor_key(t: torch.Tensor, allow_inference: bool):
    if t.layout != torch.strided:
        raise _NotCacheable
    try:
        version = t._version
    except RuntimeError:                      # inference tensor: no version counter
        if not (allow_inference and t.is_inference()):
            raise _NotCacheable
        version = None
    return (id(t), t.data_ptr(), version, tuple(t.shape), tuple(t.stride()), t.dtype, t.device)


def _key(value, allow_inference: bool = True):
    if isinstance(value, torch.Tensor):
        return _tensor_key(value, allow_inference)
    if dataclasses.is_dataclass(value) and not isinstance(value, type):
        return (type(value),) + tuple((f.name, _key(getattr(value, f.name), allow_inference))
                                      for f in dataclasses.fields(value))
    if isinstance(value, dict):
        return tuple((k, _key(v, allow_inference)) for k, v in value.items())
    if isinstance(value, (tuple, list)):
        return tuple(_key(v, allow_inference) for v in value)
    if value is None or isinstance(value, (str, int, float, bool, torch.dtype, torch.device)):
        return value
    raise _NotCacheable


def _storage_bytes(value) -> int:
    """Bytes of the storages behind ``value``'s tensors, each storage counted once."""
    seen = {}
    stack = [value]
    while stack:
        item = stack.pop()
        if isinstance(item, torch.Tensor):
            storage = item.untyped_storage()
            seen[(item.device, storage.data_ptr())] = storage.nbytes()
        elif isinstance(item, dict):
            stack.extend(item.values())
        elif isinstance(item, (tuple, list)):
            stack.extend(item)
        else:
            raise _NotCacheable
    return sum(seen.values())


def clone_tensors(value):
    if isinstance(value, torch.Tensor):
        return value.clone()
    if isinstance(value, (tuple, list)):
        return type(value)(clone_tensors(v) for v in value)
    if isinstance(value, dict):
        return {k: clone_tensors(v) for k, v in value.items()}
    return value


class _Scope:
    def __init__(self):
        self.limit = config.input_cache_max_bytes
        self.used = 0
        self.caches = set()


@contextmanager
def input_cache_scope():
    """One example's lifetime: every entry made inside is released on exit."""
    scope = _Scope()
    token = _SCOPE.set(scope)
    try:
        yield
    finally:
        for cache in list(scope.caches):
            cache.clear()
        _SCOPE.reset(token)


class InputCache:
    """Named slots sharing the active scope's byte budget (held outside ``state_dict``)."""

    def __init__(self):
        self._entries = {}

    def _drop(self, name):
        entry = self._entries.pop(name, None)
        if entry is not None:
            entry["scope"].used -= entry["bytes"]

    def clear(self):
        for name in list(self._entries):
            self._drop(name)

    def get(self, name, dependencies, owner, factory, *, modules=None, copy=None):
        scope = _SCOPE.get()
        if not config.input_cache_enabled or scope is None or owner.training or torch.is_grad_enabled():
            self.clear()
            return factory()
        members = {}                          # id -> module, in first-seen order
        for module in ((owner,) if modules is None else modules):
            for child in module.modules():
                members.setdefault(id(child), child)
        members = list(members.values())
        if any(m.training for m in members):
            self.clear()
            return factory()
        params = tuple(p for m in members for p in m.parameters(recurse=False))
        try:
            key = (scope, _key(dependencies), _key(params, allow_inference=False),
                   tuple((id(m), type(m), _key((getattr(m, "eps", None), getattr(m, "normalized_shape", None))))
                         for m in members),
                   torch.is_autocast_enabled("cpu"), torch.get_autocast_dtype("cpu"),
                   torch.is_autocast_enabled("cuda"), torch.get_autocast_dtype("cuda"),
                   config.layer_norm_implementation, config.gated_linear_unit_implementation,
                   config.dot_product_attention_implementation, config.triangle_multiplication_implementation,
                   config.packed_weight_cache_enabled)
        except _NotCacheable:
            self._drop(name)
            return factory()
        entry = self._entries.get(name)
        if entry is not None and entry["key"] == key:
            return entry["value"] if copy is None else copy(entry["value"])
        self._drop(name)
        value = factory()
        try:
            size = _storage_bytes(value)
        except _NotCacheable:
            return value
        if size > scope.limit - scope.used:
            return value
        # The entry holds its dependencies and parameters, so their addresses and ids stay
        # taken while the key is live.
        self._entries[name] = dict(key=key, value=value, deps=dependencies, params=params, scope=scope, bytes=size)
        scope.used += size
        scope.caches.add(self)
        return value if copy is None else copy(value)


def reset_input_cache(model: torch.nn.Module) -> None:
    """Releases every module's input cache (weight caches are kept)."""
    for module in model.modules():
        cache = getattr(module, "_input_cache", None)
        if isinstance(cache, InputCache):
            cache.clear()
