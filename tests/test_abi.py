"""CPU-side checks of the drop-in boundary: the C-ABI library loads, exports every symbol
include/xfold_hip.h declares, and rejects bad arguments before touching a device; the
Python mirror keeps the reference's names, parameters and guards."""

import ctypes
import json
import re
from pathlib import Path

import pytest
import torch

from tests.helpers import load_fixture
from xfold_cpu_amd.fastnn import config as fastnn_config
from xfold_cpu_amd.fastnn import native_hip as nh

HEADER = Path(__file__).resolve().parent.parent / "include" / "xfold_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(xfh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = nh.load_library()
    symbols = declared_symbols()
    assert len(symbols) >= 15
    for name in symbols:
        assert hasattr(lib, name), name
    assert set(symbols) == set(nh.SIGNATURES), "ctypes signature table and header disagree"


def test_abi_version_and_runtime_info():
    lib = nh.load_library()
    assert lib.xfh_abi_version() == nh.ABI_VERSION
    info = json.loads(nh.runtime_info())
    assert info["arch"] == "gfx950" and info["abi"] == nh.ABI_VERSION


def test_invalid_arguments_fail_before_any_launch():
    # Each call below is rejected by argument validation, so no HIP API is reached.
    with pytest.raises(ValueError, match="dtypes"):
        nh.call("xfh_layer_norm", None, 7, 4, 4, None, None, 1e-5, None, 0, None)
    with pytest.raises(ValueError, match="epilogue"):
        nh.call("xfh_linear", None, 4, None, None, 4, 4, 4, 0, None, 4, 0, 99, None, 4, 0, None)
    with pytest.raises(ValueError, match="aux"):
        nh.call("xfh_linear", None, 4, None, None, 4, 4, 4, 0, None, 4, 0, nh.EPI_MUL_SIGMOID_AUX, None, 4, 0, None)
    with pytest.raises(ValueError, match="overlap"):
        nh.call("xfh_linear_batched", None, 4, 0, None, 16, None, 0, 4, 4, 4, 2, 0, None, 4, 8, 0, None)
    with pytest.raises(ValueError, match="dtype"):
        nh.call("xfh_attention_bias_pack", None, 7, (ctypes.c_int64 * 4)(1, 1, 4, 4),
                (ctypes.c_int64 * 4)(16, 16, 4, 1), None, None)
    # A packed bias off the pipelined kernel (fp32 inputs) is refused before any launch.
    fake = ctypes.c_void_p(1 << 40)
    shape6 = (ctypes.c_int64 * 6)(1, 1, 8, 8, 8, 8)
    with pytest.raises(ValueError, match="packed bias"):
        nh.call("xfh_dot_product_attention", fake, fake, fake, nh.F32, None, 2, fake, nh.BIAS_PACKED, fake,
                nh.F32, shape6, (ctypes.c_int64 * 20)(), 1.0, None, 0, None)
    with pytest.raises(ValueError, match="head dim"):
        nh.call("xfh_grid_self_attention", None, 0, None, 2, 8, 512, 4, 0, None, None, 1e-5,
                None, None, None, None, None, None, 0, None, 0, 0, None, 0, None)
    shape = (ctypes.c_int64 * 6)(1, 1, 1, 1, 8, 8)
    strides = (ctypes.c_int64 * 20)()
    with pytest.raises(ValueError, match="dtype"):
        nh.call("xfh_dot_product_attention", None, None, None, 5, None, 2, None, 0, None, 1, shape,
                strides, 1.0, None, 0, None)
    lib = nh.load_library()
    assert "dtype" in lib.xfh_last_error().decode()


def test_workspace_too_small_is_reported():
    lib = nh.load_library()
    need = lib.xfh_triangle_multiplication_workspace_size(16, 8, nh.BF16)
    assert need > 0
    # The pointers are never dereferenced: a 16-byte workspace fails the size check before
    # any kernel is enqueued (the smallest plan needs far more).
    fake = ctypes.c_void_p(1 << 40)
    status = lib.xfh_triangle_multiplication(fake, 1, None, 2, 16, 8, 1, None, None, 1e-5, fake, fake,
                                             None, None, 1e-5, fake, fake, 1, fake, 1, 0, fake, 16,
                                             None)
    assert status == 3 and "workspace" in lib.xfh_last_error().decode()
    assert lib.xfh_grid_self_attention_workspace_size(8, 32, 4, nh.BF16) > 0
    assert lib.xfh_transition_workspace_size(64, 128, 512, nh.F32) >= 64 * (128 + 512) * 4
    assert lib.xfh_glu_packed_rows(5) == 32 and lib.xfh_glu_packed_rows(512) == 1024


def test_empty_inputs_are_no_ops():
    lib = nh.load_library()
    assert lib.xfh_layer_norm(None, 0, 0, 128, None, None, 1e-5, None, 0, None) == 0
    assert lib.xfh_linear(None, 4, None, None, 0, 4, 4, 1, None, 4, 1, 0, None, 4, 0, None) == 0
    assert lib.xfh_linear_batched(None, 4, 0, None, 16, None, 0, 4, 4, 4, 0, 1, None, 4, 16, 1, None) == 0


def test_config_defaults_to_hip_and_rejects_other_backends():
    from xfold_cpu_amd import fastnn, nn as hnn
    for name in ("layer_norm_implementation", "dot_product_attention_implementation",
                 "gated_linear_unit_implementation", "triangle_multiplication_implementation"):
        assert getattr(fastnn_config, name) == "hip"
    saved = fastnn_config.gated_linear_unit_implementation
    try:
        fastnn_config.gated_linear_unit_implementation = "torch"
        with pytest.raises(ValueError, match="only 'hip'"):
            fastnn.gated_linear_unit(torch.randn(2, 3), torch.randn(3, 4))
    finally:
        fastnn_config.gated_linear_unit_implementation = saved


def test_guards_reject_cpu_tensors_and_gradients():
    from xfold_cpu_amd import fastnn
    with pytest.raises(ValueError, match="ROCm"):
        fastnn.gated_linear_unit(torch.randn(2, 3), torch.randn(3, 4))
    with pytest.raises(ValueError, match="ROCm"):
        fastnn.dot_product_attention(torch.randn(1, 1, 2, 4), torch.randn(1, 1, 2, 4), torch.randn(1, 1, 2, 4))
    with torch.enable_grad(), pytest.raises(RuntimeError, match="inference only"):
        nh.check_gpu_inference(torch.randn(2, requires_grad=True, device="meta"))
    # A module's parameters are checked in grad mode only; a host tensor never gets a pointer.
    lin = torch.nn.Linear(2, 2)
    with torch.enable_grad(), pytest.raises(RuntimeError, match="inference only"):
        nh.check_module(lin)
    with torch.no_grad():
        nh.check_module(lin)
    with pytest.raises(ValueError, match="ROCm"):
        nh.ptr(lin.weight)
    assert nh.ptr(None) is None


def test_compute_dtype_rules():
    assert nh.compute_dtype(torch.ones(2), torch.ones(2)) == torch.float32
    with pytest.raises(ValueError, match="dtypes must match"):
        nh.compute_dtype(torch.ones(2), torch.ones(2, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        nh.compute_dtype(torch.ones(2, dtype=torch.float16))


def test_weight_cache_reuses_and_invalidates():
    weight = torch.nn.Parameter(torch.randn(7, 5))
    cache = nh.HipWeightCache()
    with torch.no_grad():
        first = cache.get(weight, torch.float32)
        assert first is cache.get(weight, torch.float32)
        weight.add_(1)
        updated = cache.get(weight, torch.float32)
        assert updated is not first
        torch.testing.assert_close(updated, weight)
        assert cache.get(weight, torch.bfloat16).dtype == torch.bfloat16
    with torch.inference_mode():
        cache.get(torch.randn(5, 7), torch.float32)
    assert cache._key is None


def test_derived_weight_rebuilds_when_a_source_changes():
    """Weights derived from several parameters (stacked projections, folded LayerNorm
    weights) are built once and rebuilt when any source is updated in place."""
    module = torch.nn.Module()
    a, b = torch.nn.Parameter(torch.randn(3, 4)), torch.nn.Parameter(torch.randn(2, 4))
    calls = []

    def build(*ws):
        calls.append(1)
        return torch.cat([w.detach() for w in ws], dim=0)

    with torch.no_grad():
        first = nh.derived_weight(module, "stack", [a, b], build)
        assert nh.derived_weight(module, "stack", [a, b], build) is first and len(calls) == 1
        b.mul_(2)
        second = nh.derived_weight(module, "stack", [a, b], build)
        assert second is not first and len(calls) == 2
        torch.testing.assert_close(second, torch.cat([a, b]))
        assert nh.derived_weight(module, "other", [a], build) is not second and len(calls) == 3
    with torch.inference_mode():
        c = torch.randn(2, 4)
        nh.derived_weight(module, "inference", [c], build)
        nh.derived_weight(module, "inference", [c], build)
    assert len(calls) == 5                            # inference tensors are never cached


@pytest.mark.parametrize("fixture,cls", [
    ("pairformer_block", "PairformerBlock"), ("diffusion_transformer", "DiffusionTransformer"),
    ("grid_attention_start", "GridSelfAttention"), ("self_attention_cond", "SelfAttention"),
    ("diffusion_transition", "DiffusionTransition"), ("transition", "Transition")])
def test_modules_keep_the_reference_parameter_names(fixture, cls):
    """state_dict keys of the HIP modules equal those of the reference modules (recorded
    in the golden fixtures), so checkpoints load unchanged."""
    from xfold_cpu_amd import nn as hnn
    meta, _, params, _ = load_fixture(fixture)
    module = getattr(hnn, cls)(**meta["args"])
    module.load_state_dict(params, strict=True)
