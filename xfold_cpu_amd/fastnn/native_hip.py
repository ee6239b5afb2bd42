"""ctypes bridge to libxfold_hip.so (the MI355X backend), mirroring the reference's
native bridge ``xfold/fastnn/native.py:1-70``:

* :func:`load_library`    ~ ``load_native_operator`` (``native.py:7-18``): loads once,
                            checks the ABI version and every exported symbol, and fails
                            loudly (RuntimeError) when the library is missing. There is no
                            fallback to another implementation.
* :func:`check_gpu_inference` ~ ``check_cpu_inference`` (``native.py:21-28``) for ROCm
                            tensors (``device.type == 'cuda'`` under PyTorch-ROCm).
* :func:`compute_dtype`   ~ ``compute_dtype`` (``native.py:31-43``) with the CUDA/HIP
                            autocast state instead of the CPU one.
* :class:`HipWeightCache` ~ ``GLUWeightCache`` (``xfold/fastnn/gated_linear_unit.py:6-48``):
                            one device copy per weight version in the compute dtype, and
                            the packed GLU layout.

Torch is used here only for device memory, streams and dtype bookkeeping; all arithmetic
runs in the library's HIP kernels.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path
from typing import Optional

import torch

LIBRARY_PATH = Path(__file__).resolve().parent.parent / "lib" / "libxfold_hip.so"
ABI_VERSION = 9

F32, BF16, BOOL = 0, 1, 2
BIAS_PACKED = 3                 # bias 'dtype' of a packed fp32 block (times log2(e))
BIAS_PACKED_BF16 = 4            # bias 'dtype' of a packed bf16 block (natural units)
EPI_STORE, EPI_MUL_SIGMOID_AUX, EPI_SIGMOID_MUL_AUX, EPI_ACCUMULATE, EPI_MUL_SIGMOID_AUX_ACCUMULATE = range(5)

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_pi64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must match include/xfold_hip.h.
SIGNATURES = {
    "xfh_abi_version": (_i, []),
    "xfh_runtime_info": (ctypes.c_char_p, []),
    "xfh_last_error": (ctypes.c_char_p, []),
    "xfh_set_kernel_timing": (None, [_i]),
    "xfh_kernel_timing_read": (_i, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), _pi64]),
    "xfh_kernel_timing_read_work": (_i, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), _pi64,
                                         ctypes.POINTER(ctypes.c_double)]),
    "xfh_layer_norm": (_i, [_p, _i, _i64, _i64, _p, _p, _f, _p, _i, _p]),
    "xfh_adaptive_layer_norm": (_i, [_p, _i, _i64, _i64, _p, _p, _i, _i64, _f, _p, _i, _p]),
    "xfh_linear": (_i, [_p, _i64, _p, _p, _i64, _i64, _i64, _i, _p, _i64, _i, _i, _p, _i64, _i64, _p]),
    "xfh_linear_batched": (_i, [_p, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i, _p, _i64, _i64, _i, _p]),
    "xfh_glu_packed_rows": (_i64, [_i64]),
    "xfh_glu_pack_weight": (_i, [_p, _i64, _i64, _i, _p, _p]),
    "xfh_gated_linear_unit": (_i, [_p, _p, _i64, _i64, _i64, _i, _p, _i, _p]),
    "xfh_dot_product_attention_workspace_size": (_i64, [_pi64, _i]),
    "xfh_dot_product_attention": (_i, [_p, _p, _p, _i, _p, _i, _p, _i, _p, _i, _pi64, _pi64, _f, _p, _i64, _p]),
    "xfh_attention_max_keys": (_i64, []),
    "xfh_attention_bias_pack": (_i, [_p, _i, _pi64, _pi64, _p, _p]),
    "xfh_attention_operands_size": (_i, [_i64, _i64, _i64, _i64, _pi64]),
    "xfh_attention_project": (_i, [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, _p, _p, _p, _p, _p]),
    "xfh_attention_mask_words": (_i, [_p, _i, _i64, _i64, _i64, _p, _p]),
    "xfh_attention_operands": (_i, [_p, _p, _p, _p, _i, _p, _i, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "xfh_pair_attention_bias": (_i, [_p, _i, _i64, _i64, _p, _p, _f, _p, _i, _i64, _p, _i, _p]),
    "xfh_triangle_multiplication_workspace_size": (_i64, [_i64, _i64, _i]),
    "xfh_triangle_multiplication": (_i, [_p, _i, _p, _i, _i64, _i64, _i, _p, _p, _f, _p, _p, _p, _p,
                                         _f, _p, _p, _i, _p, _i, _i, _p, _i64, _p]),
    "xfh_triangle_multiplication_noalloc": (_i, [_p, _i, _p, _i, _i64, _i64, _i, _p, _p, _f, _p, _p, _p, _p,
                                                 _f, _p, _p, _i, _p, _i, _i, _p]),
    "xfh_grid_self_attention_workspace_size": (_i64, [_i64, _i64, _i64, _i]),
    "xfh_grid_self_attention": (_i, [_p, _i, _p, _i, _i64, _i64, _i64, _i, _p, _p, _f, _p, _p, _p,
                                     _p, _p, _p, _i, _p, _i, _i, _p, _i64, _p]),
    "xfh_transition_workspace_size": (_i64, [_i64, _i64, _i64, _i]),
    "xfh_transition": (_i, [_p, _i, _i64, _i64, _i64, _p, _p, _f, _p, _p, _i, _p, _i, _i, _p, _i64, _p]),
    "xfh_transition_pair_bias": (_i, [_p, _i64, _i64, _i64, _p, _p, _f, _p, _p, _p, _p, _f, _p, _i64, _p, _p]),
    "xfh_outer_product_mean_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _i]),
    "xfh_outer_product_mean": (_i, [_p, _i, _p, _i, _i64, _i64, _i64, _i64, _i64, _p, _p, _f, _p, _p, _p, _f,
                                    _i, _p, _i, _i, _p, _i64, _p]),
    "xfh_msa_attention_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _i64, _i]),
    "xfh_msa_attention": (_i, [_p, _i, _p, _i, _p, _i, _i64, _i64, _i64, _i64, _i64, _p, _p, _f, _p, _p, _f,
                               _p, _p, _p, _p, _i, _p, _i, _i, _p, _i64, _p]),
    "xfh_cross_attention_bias": (_i, [_p, _i, _pi64, _p, _i, _p, _i, _i64, _i64, _i64, _i64, _p, _p]),
    "xfh_convert": (_i, [_p, _i, _p, _i, _i64, _p]),
}


class HipBackendError(RuntimeError):
    """A libxfold_hip call returned an error status."""


@functools.lru_cache(maxsize=None)
def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """Load libxfold_hip.so once; raise RuntimeError if it is absent or incomplete."""
    lib_path = Path(path or os.environ.get("XFOLD_HIP_LIBRARY", LIBRARY_PATH))
    if not lib_path.exists():
        raise RuntimeError(
            f"The 'hip' backend needs {lib_path}; build it with `python -m xfold_cpu_amd._build` "
            "(hipcc, gfx950) before selecting 'hip'.")
    lib = ctypes.CDLL(str(lib_path))
    missing = [name for name in SIGNATURES if not hasattr(lib, name)]
    if missing:
        raise RuntimeError(f"Rebuild libxfold_hip.so: missing symbols {missing}.")
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.xfh_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libxfold_hip.so ABI {version} != expected {ABI_VERSION}; rebuild it.")
    return lib


def call(name: str, *args) -> None:
    lib = load_library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.xfh_last_error().decode()
        if status in (1, 2):
            raise ValueError(f"{name}: {message}")
        raise HipBackendError(f"{name} failed ({status}): {message}")


def set_kernel_timing(enable: bool) -> None:
    load_library().xfh_set_kernel_timing(int(enable))


def kernel_timing_read(name: str):
    """(total milliseconds, launches) recorded for ``name`` since the last read."""
    total, count = ctypes.c_double(), ctypes.c_int64()
    call("xfh_kernel_timing_read", name.encode(), ctypes.byref(total), ctypes.byref(count))
    return total.value, count.value


def kernel_timing_read_work(name: str):
    """(total milliseconds, launches, total declared FLOPs) recorded for ``name`` since the
    last read."""
    total, count, work = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double()
    call("xfh_kernel_timing_read_work", name.encode(), ctypes.byref(total), ctypes.byref(count), ctypes.byref(work))
    return total.value, count.value, work.value


@functools.lru_cache(maxsize=None)
def attention_max_keys() -> int:
    """Largest key count of the pipelined attention kernel, hence of a packed bias."""
    return int(load_library().xfh_attention_max_keys())


def runtime_info() -> str:
    return load_library().xfh_runtime_info().decode()


# ------------------------------------------------------------------------- tensor helpers

def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return F32
    if dtype == torch.bfloat16:
        return BF16
    if dtype in (torch.bool, torch.uint8):
        return BOOL
    raise ValueError(f"The 'hip' backend supports FP32/BF16 tensors (and bool masks), got {dtype}.")


def check_gpu_inference(*tensors) -> None:
    """Device, layout and inference-only guards (reference ``native.py:21-28``)."""
    for tensor in tensors:
        if tensor is None:
            continue
        if torch.is_grad_enabled() and tensor.requires_grad:
            raise RuntimeError("The 'hip' backend supports inference only; disable gradients.")
        if tensor.device.type != "cuda" or tensor.layout != torch.strided:
            raise ValueError("The 'hip' backend requires strided ROCm (cuda) tensors.")


def compute_dtype(x: torch.Tensor, *weights: torch.Tensor) -> torch.dtype:
    """Compute dtype per reference ``native.py:31-43``, reading the CUDA autocast state."""
    for tensor in (x, *weights):
        if tensor.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("The 'hip' backend supports FP32/BF16 only.")
    if torch.is_autocast_enabled("cuda"):
        dtype = torch.get_autocast_dtype("cuda")
    else:
        dtype = x.dtype
        if any(w.dtype != dtype for w in weights):
            raise ValueError("Input/weight dtypes must match outside autocast.")
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("The 'hip' backend supports FP32/BF16 autocast only.")
    return dtype


def check_module(module: torch.nn.Module) -> None:
    """Inference-only guard for a module's parameters (reference ``native.py:21-28``): a
    parameter that requires grad matters only in grad mode, so the walk over them happens
    only then; their device is checked where their pointers are taken (:func:`ptr`)."""
    if torch.is_grad_enabled():
        check_gpu_inference(*module.parameters())


def ptr(tensor: Optional[torch.Tensor]) -> Optional[int]:
    """Device address of a tensor handed to the library; a host tensor is refused here."""
    if tensor is None:
        return None
    if not tensor.is_cuda:
        raise ValueError("The 'hip' backend requires strided ROCm (cuda) tensors.")
    return tensor.data_ptr()


def stream_of(device: torch.device) -> int:
    """The current stream of ``device`` as a raw hipStream_t."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch memory (PyTorch caching allocator); the library allocates none."""
    if nbytes < 0:
        raise ValueError("invalid workspace request")
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def mask_arg(mask: Optional[torch.Tensor], shape) -> tuple:
    """(tensor, dtype code) of a contiguous mask broadcast to ``shape`` (kept alive by caller)."""
    if mask is None:
        return None, BOOL
    if mask.dtype not in (torch.float32, torch.bfloat16, torch.bool, torch.uint8):
        raise ValueError("masks must be bool/uint8/float32/bfloat16")
    if tuple(mask.shape) != tuple(shape):
        mask = mask.expand(shape)
    return mask.contiguous(), dtype_code(mask.dtype)


class HipWeightCache:
    """Device copy of one weight in a compute dtype, re-made when the weight changes.

    Keyed like the reference ``GLUWeightCache`` (``gated_linear_unit.py:15-30``) on
    (data_ptr, _version, shape, stride, dtype, device, compute dtype, layout); tensors
    without a version counter (inference tensors) are never cached. ``layout`` is
    ``"plain"`` (contiguous copy) or ``"glu"`` (the packed gate/value layout).
    """

    def __init__(self):
        self._key = None
        self._source = None
        self._value = None

    def clear(self):
        self._key = self._source = self._value = None

    def get(self, weight: torch.Tensor, dtype: torch.dtype, layout: str = "plain") -> torch.Tensor:
        try:
            version = weight._version
        except RuntimeError:
            self.clear()
            return _prepare(weight, dtype, layout)
        key = (weight.data_ptr(), version, weight.shape, weight.stride(), weight.dtype, weight.device, dtype, layout)
        if self._key != key:
            self._value = _prepare(weight, dtype, layout)
            self._source = weight          # keeps the address from being reused
            self._key = key
        return self._value


def _prepare(weight: torch.Tensor, dtype: torch.dtype, layout: str) -> torch.Tensor:
    w = weight.detach().to(dtype=dtype).contiguous()
    if layout == "plain":
        return w
    if layout == "glu":
        # w is transition1.weight: [2F, K], rows [0, F) = SiLU gate.
        rows2f, k = w.shape
        f = rows2f // 2
        lib = load_library()
        packed = torch.empty((lib.xfh_glu_packed_rows(f), k), dtype=dtype, device=w.device)
        call("xfh_glu_pack_weight", ptr(w), f, k, dtype_code(dtype), ptr(packed), stream_of(w.device))
        return packed
    raise ValueError(f"unknown weight layout {layout}")


def module_cache(module: torch.nn.Module, name: str) -> HipWeightCache:
    """Per-module weight caches, held outside ``state_dict`` (like ``_native_weights``)."""
    caches = module.__dict__.setdefault("_hip_weight_caches", {})
    cache = caches.get(name)
    if cache is None:
        cache = caches[name] = HipWeightCache()
    return cache


def linear_weight(module: torch.nn.Module, name: str, dtype: torch.dtype, layout: str = "plain"):
    """Device copy of ``module.<name>.weight`` ([out, in]) in ``dtype``."""
    return module_cache(module, name).get(getattr(module, name).weight, dtype, layout)


class FusedWeightCache:
    """Row-concatenation of several weights ([out_i, in] -> [sum out_i, in]) in one dtype,
    re-made when any source weight changes (same keys as :class:`HipWeightCache`)."""

    def __init__(self):
        self._key = None
        self._sources = None
        self._value = None

    def get(self, weights, dtype: torch.dtype) -> torch.Tensor:
        try:
            key = tuple((w.data_ptr(), w._version, w.shape, w.stride(), w.dtype, w.device)
                        for w in weights) + (dtype,)
        except RuntimeError:
            self._key = self._sources = self._value = None
            return torch.cat([w.detach().to(dtype) for w in weights], dim=0).contiguous()
        if self._key != key:
            self._value = torch.cat([w.detach().to(dtype) for w in weights], dim=0).contiguous()
            self._sources = tuple(weights)
            self._key = key
        return self._value


def fused_linear_weight(module: torch.nn.Module, names, dtype: torch.dtype) -> torch.Tensor:
    caches = module.__dict__.setdefault("_hip_weight_caches", {})
    tag = "fused:" + ",".join(names)
    cache = caches.get(tag)
    if cache is None:
        cache = caches[tag] = FusedWeightCache()
    return cache.get([getattr(module, n).weight for n in names], dtype)


class DerivedWeightCache:
    """A tensor built from several parameters by ``build(*sources)`` (a one-time weight
    preparation), re-made when any source changes (same keys as :class:`HipWeightCache`;
    never cached when a source is an inference tensor)."""

    def __init__(self):
        self._key = None
        self._sources = None
        self._value = None

    def get(self, sources, build):
        try:
            key = tuple((t.data_ptr(), t._version, t.shape, t.stride(), t.dtype, t.device) for t in sources)
        except RuntimeError:
            self._key = self._sources = self._value = None
            return build(*sources)
        if self._key != key:
            self._value = build(*sources)
            self._sources = tuple(sources)
            self._key = key
        return self._value


def derived_weight(module: torch.nn.Module, tag: str, sources, build):
    caches = module.__dict__.setdefault("_hip_weight_caches", {})
    cache = caches.get(tag)
    if cache is None:
        cache = caches[tag] = DerivedWeightCache()
    return cache.get(list(sources), build)


def fp32_param(module: torch.nn.Module, name: str, param: Optional[torch.Tensor]):
    """LayerNorm affine parameters as contiguous fp32 (None stays None)."""
    if param is None:
        return None
    if param.dtype == torch.float32 and param.is_contiguous():
        return param.detach()
    return module_cache(module, name).get(param, torch.float32)
