"""Per-example memo for the hip DiffusionTransformer's static inputs.

What it keeps: the packed pair logits of every super-block (the only entry the hip
DiffusionTransformer makes), computed from ``pair_cond`` and weights that do not change
while one example is sampled, so the sampler's repeated calls skip the pair-logit pass
(the reuse ``xfold/nn/diffusion_transformer.py:255-265`` asks of its module cache).

Interface: ``input_cache_scope()``, ``InputCache.get(name, dependencies, owner, factory,
*, modules=None, copy=None)`` and ``reset_input_cache(model)`` have the names and argument
meaning of the reference's (``xfold/nn/cache.py:84-151``), so a module can carry either
class and callers open scopes the same way; ``config.input_cache_enabled`` and
``config.input_cache_max_bytes`` gate and bound it as in the reference.

Design (this module's own):
  * An entry stores the objects it was computed from: the dependency tensors, the
    parameters of the listed modules, and a *stamp* of each (version counter, address,
    shape, strides, dtype, device), plus a *context* tuple (the non-tensor leaves of the
    dependencies, the modules' ``eps`` and ``normalized_shape``, the autocast state of
    both device types and the backend switches). It is valid while every tensor passed now
    is the very object it holds (``is``, so no id or address reuse can alias) with an
    unchanged stamp, and the context compares equal. Holding the objects keeps them alive
    for as long as the entry does.
  * A tensor without a version counter (created under ``torch.inference_mode``) cannot
    show an in-place update: it is accepted as an input feature, which the scope declares
    immutable, and never as a weight; a module with such a weight is not memoised.
  * ``ExampleScope`` is the byte ledger of one example: each entry is charged the full
    storages its value keeps alive (shared storages once). A value that would overdraw the
    budget is returned without being kept. Closing the scope, normally or by an exception,
    releases every entry it paid for.
  * Nothing is kept outside a scope, with grad mode on, or while the owner or a listed
    module is training; such a call also drops what the cache held.
"""

from __future__ import annotations

import dataclasses
from contextvars import ContextVar
from typing import Any, Callable, Dict, List, Optional, Tuple

import torch
from torch.utils._pytree import tree_map

from ..fastnn import config

_ACTIVE: ContextVar[Optional["ExampleScope"]] = ContextVar("xfold_cpu_amd_example_scope", default=None)


class _Refused(Exception):
    """The request names something the memo cannot stamp (a sparse tensor, an unknown
    leaf type, or a versionless weight)."""


def _stamp(t: torch.Tensor, weight: bool) -> tuple:
    if t.layout != torch.strided:
        raise _Refused
    try:
        version = t._version
    except RuntimeError:                      # inference tensor: no version counter
        if weight or not t.is_inference():
            raise _Refused
        version = -1
    return (version, t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype, t.device)


_LEAF_TYPES = (str, int, float, bool, torch.dtype, torch.device, type(None))


def _split(value: Any, tensors: List[torch.Tensor]) -> Any:
    """Moves every tensor of ``value`` (in visiting order) to ``tensors`` and returns the
    rest of its structure, comparable with ``==``, with each tensor's slot marked."""
    if isinstance(value, torch.Tensor):
        tensors.append(value)
        return ("<tensor>", len(tensors) - 1)
    if isinstance(value, _LEAF_TYPES):
        return value
    if isinstance(value, (list, tuple)):
        return (type(value).__name__, tuple(_split(v, tensors) for v in value))
    if isinstance(value, dict):
        return ("dict", tuple((k, _split(v, tensors)) for k, v in value.items()))
    if dataclasses.is_dataclass(value) and not isinstance(value, type):
        return (type(value), tuple((f.name, _split(getattr(value, f.name), tensors))
                                   for f in dataclasses.fields(value)))
    raise _Refused


def _storage_footprint(value: Any) -> int:
    """Bytes of the distinct storages that ``value``'s tensors keep alive."""
    tensors: List[torch.Tensor] = []
    _split(value, tensors)
    sizes: Dict[tuple, int] = {}
    for t in tensors:
        storage = t.untyped_storage()
        sizes[(t.device, storage.data_ptr())] = storage.nbytes()
    return sum(sizes.values())


def clone_tensors(value: Any) -> Any:
    """A copy of ``value`` whose tensors are fresh clones (a ``copy=`` argument for
    ``InputCache.get`` when the caller updates the returned tensors in place)."""
    return tree_map(lambda v: v.clone() if isinstance(v, torch.Tensor) else v, value)


class ExampleScope:
    """Byte ledger and lifetime of one example's memoised inputs (a context manager)."""

    def __init__(self, limit: Optional[int] = None):
        self.limit = config.input_cache_max_bytes if limit is None else limit
        self.used = 0
        self._holders: Dict[Tuple[int, str], "InputCache"] = {}
        self._token = None

    def charge(self, cache: "InputCache", name: str, nbytes: int) -> bool:
        if nbytes > self.limit - self.used:
            return False
        self.used += nbytes
        self._holders[(id(cache), name)] = cache
        return True

    def refund(self, cache: "InputCache", name: str, nbytes: int) -> None:
        self.used -= nbytes
        self._holders.pop((id(cache), name), None)

    def close(self) -> None:
        for (_, name), cache in list(self._holders.items()):
            cache.release(name)
        self._holders.clear()

    def __enter__(self) -> "ExampleScope":
        self._token = _ACTIVE.set(self)
        return self

    def __exit__(self, *exc) -> None:
        try:
            self.close()
        finally:
            _ACTIVE.reset(self._token)


def input_cache_scope() -> ExampleScope:
    """Opens one example's scope: ``with input_cache_scope(): ...``. Entries made inside
    are released when it closes (also on an exception)."""
    return ExampleScope()


@dataclasses.dataclass
class _Entry:
    scope: ExampleScope
    value: Any
    held: Tuple[torch.Tensor, ...]            # dependency tensors, then parameters
    stamps: Tuple[tuple, ...]
    context: tuple
    nbytes: int

    def matches(self, scope, held, context) -> bool:
        if scope is not self.scope or context != self.context or len(held) != len(self.held):
            return False
        for now, kept, stamp in zip(held, self.held, self.stamps):
            if now is not kept:
                return False
            try:
                version = now._version
            except RuntimeError:
                version = -1
            if (version, now.data_ptr(), tuple(now.shape), tuple(now.stride()), now.dtype, now.device) != stamp:
                return False
        return True


def _members(owner: torch.nn.Module, modules) -> List[torch.nn.Module]:
    roots = (owner,) if modules is None else (modules if isinstance(modules, (list, tuple)) else (modules,))
    seen: Dict[int, torch.nn.Module] = {}
    for root in roots:
        for m in root.modules():
            seen.setdefault(id(m), m)
    return list(seen.values())


def _environment() -> tuple:
    return (torch.is_autocast_enabled("cuda"), torch.get_autocast_dtype("cuda"),
            torch.is_autocast_enabled("cpu"), torch.get_autocast_dtype("cpu"),
            config.layer_norm_implementation, config.gated_linear_unit_implementation,
            config.dot_product_attention_implementation, config.triangle_multiplication_implementation,
            config.packed_weight_cache_enabled)


class InputCache:
    """Named memo slots of one module; the active ``ExampleScope`` pays for them. Kept as a
    plain attribute, never in ``state_dict``."""

    def __init__(self):
        self._entries: Dict[str, _Entry] = {}

    def release(self, name: str) -> None:
        entry = self._entries.pop(name, None)
        if entry is not None:
            entry.scope.refund(self, name, entry.nbytes)

    def clear(self) -> None:
        for name in list(self._entries):
            self.release(name)

    def get(self, name: str, dependencies: Any, owner: torch.nn.Module, factory: Callable[[], Any], *,
            modules=None, copy: Optional[Callable[[Any], Any]] = None) -> Any:
        scope = _ACTIVE.get()
        members = _members(owner, modules)
        if (scope is None or not config.input_cache_enabled or torch.is_grad_enabled()
                or owner.training or any(m.training for m in members)):
            self.clear()
            return factory()
        deps: List[torch.Tensor] = []
        try:
            shape = _split(dependencies, deps)
            params = list({id(p): p for m in members for p in m.parameters(recurse=False)}.values())
            stamps = tuple(_stamp(t, weight=False) for t in deps) + tuple(_stamp(p, weight=True) for p in params)
            settings = tuple((type(m).__name__, getattr(m, "eps", None),
                              tuple(getattr(m, "normalized_shape", ()) or ())) for m in members)
        except _Refused:
            self.release(name)
            return factory()
        held = tuple(deps) + tuple(params)
        context = (shape, settings, _environment())
        entry = self._entries.get(name)
        if entry is not None and entry.matches(scope, held, context):
            return entry.value if copy is None else copy(entry.value)
        self.release(name)
        value = factory()
        try:
            nbytes = _storage_footprint(value)
        except _Refused:
            return value
        if scope.charge(self, name, nbytes):
            self._entries[name] = _Entry(scope, value, held, stamps, context, nbytes)
        return value if copy is None else copy(value)


def reset_input_cache(model: torch.nn.Module) -> None:
    """Releases the memo slots of every module of ``model`` (weight caches are separate and
    stay)."""
    for m in model.modules():
        memo = m.__dict__.get("_input_cache")
        if isinstance(memo, InputCache):
            memo.clear()
