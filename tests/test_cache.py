"""The hip DiffusionTransformer's input cache (xfold_cpu_amd/nn/cache.py) on the CPU: the
reference's own cache cases (tests/test_cpu_runtime.py:127-190 in the reference) —
reuse within a scope, invalidation by an in-place feature or weight update, copies,
the shared byte budget, release on scope exit and on exceptions, no caching in training
mode, and versionless (inference) tensors cached as features but never as weights."""

import pytest
import torch
import torch.nn as nn

from xfold_cpu_amd.fastnn import config
from xfold_cpu_amd.nn.cache import InputCache, input_cache_scope, reset_input_cache


@pytest.fixture(autouse=True)
def cache_config():
    saved = (config.input_cache_enabled, config.input_cache_max_bytes)
    config.input_cache_enabled = True
    yield
    config.input_cache_enabled, config.input_cache_max_bytes = saved


def test_reuses_and_invalidates_on_feature_and_weight_updates():
    owner, cache, feature = nn.Linear(3, 3).eval(), InputCache(), torch.randn(2, 3)
    calls = []

    def factory():
        calls.append(1)
        return owner(feature)
    with torch.no_grad(), input_cache_scope():
        first = cache.get("x", (feature,), owner, factory)
        assert cache.get("x", (feature,), owner, factory) is first
        feature.add_(1)
        second = cache.get("x", (feature,), owner, factory)
        assert second is not first
        owner.weight.add_(1)
        assert cache.get("x", (feature,), owner, factory) is not second
        assert len(calls) == 3
    assert not cache._entries


def test_copy_budget_training_and_exception_cleanup():
    owner, cache, feature = nn.Linear(3, 3).eval(), InputCache(), torch.randn(2, 3)
    calls = []

    def factory():
        calls.append(1)
        return feature * 2
    with torch.no_grad(), input_cache_scope():
        cache.get("x", (feature,), owner, factory, copy=torch.clone).zero_()
        torch.testing.assert_close(cache.get("x", (feature,), owner, factory, copy=torch.clone), feature * 2)
        assert len(calls) == 1
    config.input_cache_max_bytes = 1
    with torch.no_grad(), input_cache_scope():
        cache.get("x", (feature,), owner, factory)
        cache.get("x", (feature,), owner, factory)
        assert not cache._entries
    config.input_cache_max_bytes = 4096
    with pytest.raises(RuntimeError, match="test exception"), torch.no_grad(), input_cache_scope():
        cache.get("x", (feature,), owner, factory)
        raise RuntimeError("test exception")
    assert not cache._entries
    owner.train()
    with torch.no_grad(), input_cache_scope():
        cache.get("x", (feature,), owner, factory)
        assert not cache._entries


def test_no_caching_outside_a_scope_or_when_disabled_or_with_grad():
    owner, cache, feature = nn.Linear(3, 3).eval(), InputCache(), torch.randn(2, 3)
    calls = []

    def factory():
        calls.append(1)
        return feature * 2
    with torch.no_grad():
        cache.get("x", (feature,), owner, factory)
        cache.get("x", (feature,), owner, factory)
    with input_cache_scope():                        # grad mode on
        cache.get("x", (feature,), owner, factory)
    config.input_cache_enabled = False
    with torch.no_grad(), input_cache_scope():
        cache.get("x", (feature,), owner, factory)
    assert len(calls) == 4 and not cache._entries


def test_inference_features_cache_but_versionless_weights_do_not():
    owner = nn.Linear(3, 3).eval()
    cache, calls = InputCache(), []
    with torch.inference_mode(), input_cache_scope():
        feature = torch.ones(2, 3)

        def factory():
            calls.append(1)
            return feature * 2
        assert cache.get("x", (feature,), owner, factory) is cache.get("x", (feature,), owner, factory)
        assert len(calls) == 1
        versionless_owner = nn.Linear(3, 3).eval()
        cache.get("y", (feature,), versionless_owner, factory)
        cache.get("y", (feature,), versionless_owner, factory)
        assert len(calls) == 3


def test_reset_input_cache_releases_module_caches():
    model = nn.Sequential(nn.Linear(3, 3)).eval()
    model[0]._input_cache = InputCache()
    feature = torch.randn(2, 3)
    with torch.no_grad(), input_cache_scope():
        model[0]._input_cache.get("x", (feature,), model[0], lambda: feature * 2)
        assert model[0]._input_cache._entries
        reset_input_cache(model)
        assert not model[0]._input_cache._entries


def test_a_new_tensor_at_the_same_address_or_another_autocast_state_is_a_miss():
    """Validity is the held object itself (not its id or address) with an unchanged
    stamp, plus the autocast state and module settings the value was computed under."""
    owner, cache, feature = nn.Linear(3, 3).eval(), InputCache(), torch.randn(2, 3)
    calls = []

    def factory():
        calls.append(1)
        return feature * 2
    with torch.no_grad(), input_cache_scope() as scope:
        cache.get("x", (feature, 4), owner, factory)
        alias = feature.view(2, 3)                   # same storage and address, new object
        cache.get("x", (alias, 4), owner, factory)
        cache.get("x", (alias, 5), owner, factory)   # a non-tensor leaf changed
        with torch.autocast("cpu", dtype=torch.bfloat16):
            cache.get("x", (alias, 5), owner, factory)
        assert len(calls) == 4
        assert scope.used == feature.untyped_storage().nbytes()
    assert scope.used == 0 and not cache._entries


def test_entries_are_charged_per_distinct_storage():
    owner, cache = nn.Linear(3, 3).eval(), InputCache()
    base = torch.zeros(64)
    with torch.no_grad(), input_cache_scope() as scope:
        cache.get("views", (), owner, lambda: (base[:8], base[8:], {"again": base}))
        assert scope.used == base.untyped_storage().nbytes()
        cache.get("other", (), owner, lambda: torch.zeros(16))
        assert scope.used == base.untyped_storage().nbytes() + 64
        reset_input_cache(nn.Sequential())           # no module of this model holds them
        assert scope.used > 0
