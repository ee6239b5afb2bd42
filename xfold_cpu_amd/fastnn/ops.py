"""HIP operator wrappers over libxfold_hip.so (tensor checks, dtype resolution, launch).

Each function validates its torch tensors, resolves the compute dtype (CUDA/HIP autocast
state, as the reference resolves the CPU one in ``xfold/fastnn/native.py:31-43``),
allocates outputs and workspaces with the PyTorch caching allocator, and enqueues the
library call on the current stream. None of them computes anything with torch.
"""

from __future__ import annotations

import collections
import ctypes
import threading
from typing import Optional

import torch

from . import native_hip as nh


def _out_dtype_for_norm(x: torch.Tensor) -> torch.dtype:
    # CUDA autocast runs layer_norm in fp32 (its fp32 op list); outside autocast the
    # output keeps the input dtype, as F.layer_norm does.
    return torch.float32 if torch.is_autocast_enabled("cuda") else x.dtype


def layer_norm(x: torch.Tensor, normalized_shape, weight: Optional[torch.Tensor],
               bias: Optional[torch.Tensor], eps: float, out_dtype: Optional[torch.dtype] = None,
               owner: Optional[torch.nn.Module] = None) -> torch.Tensor:
    """F.layer_norm over the trailing ``normalized_shape`` (``xfold/fastnn/layer_norm.py:56-59``)."""
    nh.check_gpu_inference(x, weight, bias)
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("The 'hip' LayerNorm supports FP32/BF16 inputs.")
    shape = tuple(normalized_shape) if not isinstance(normalized_shape, int) else (normalized_shape,)
    if tuple(x.shape[len(x.shape) - len(shape):]) != shape:
        raise ValueError(f"LayerNorm: input shape {tuple(x.shape)} does not end with {shape}.")
    cols = 1
    for s in shape:
        cols *= s
    x_c = x.contiguous()
    rows = x_c.numel() // cols if cols else 0
    out_dtype = out_dtype or _out_dtype_for_norm(x)
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    w = _fp32(weight, owner, "ln_weight")
    b = _fp32(bias, owner, "ln_bias")
    nh.call("xfh_layer_norm", nh.ptr(x_c), nh.dtype_code(x.dtype), rows, cols, nh.ptr(w), nh.ptr(b),
            float(eps), nh.ptr(y), nh.dtype_code(out_dtype), nh.stream_of(x.device))
    return y


def _fp32(param, owner, name):
    if param is None:
        return None
    if param.dtype == torch.float32 and param.is_contiguous():
        return param.detach()
    if owner is not None:
        return nh.module_cache(owner, name).get(param, torch.float32)
    return param.detach().to(torch.float32).contiguous()


def adaptive_layer_norm(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float,
                        out_dtype: torch.dtype) -> torch.Tensor:
    """sigmoid(scale) * LN_noaffine(x) + shift; scale/shift [cond_rows, C] broadcast over
    leading sample dims (``xfold/nn/diffusion_transformer.py:57-62``)."""
    cols = x.shape[-1]
    x_c = x.contiguous()
    rows = x_c.numel() // cols
    cond_rows = scale.numel() // cols
    if scale.shape != shift.shape or rows % max(cond_rows, 1):
        raise ValueError("adaptive LayerNorm: condition rows must tile the input rows")
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    nh.call("xfh_adaptive_layer_norm", nh.ptr(x_c), nh.dtype_code(x.dtype), rows, cols,
            nh.ptr(scale), nh.ptr(shift), nh.dtype_code(scale.dtype), cond_rows, float(eps),
            nh.ptr(y), nh.dtype_code(out_dtype), nh.stream_of(x.device))
    return y


def as_dtype(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """x contiguous in ``dtype`` (f32/bf16); a dtype change runs in this library's kernel."""
    if x.dtype == dtype:
        return x.contiguous()
    if x.dtype not in (torch.float32, torch.bfloat16) or dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"as_dtype: {x.dtype} -> {dtype} (f32/bf16 only)")
    x_c = x.contiguous()
    y = torch.empty(x.shape, dtype=dtype, device=x.device)
    nh.call("xfh_convert", nh.ptr(x_c), nh.dtype_code(x.dtype), nh.ptr(y), nh.dtype_code(dtype), x_c.numel(),
            nh.stream_of(x.device))
    return y


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], dtype: torch.dtype,
           out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
           epilogue: int = nh.EPI_STORE, aux: Optional[torch.Tensor] = None,
           aux_rows: int = 0) -> torch.Tensor:
    """``out = epilogue(x @ weight^T + bias)`` with weight already in the compute dtype.

    x is cast to the compute dtype if needed (the autocast cast of ``nn.Linear``). ``out``
    may be given (e.g. the residual stream for the accumulate epilogues).
    """
    k = x.shape[-1]
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError(f"linear: weight {tuple(weight.shape)} does not match input dim {k}")
    x_c = as_dtype(x, dtype)
    m = x_c.numel() // k if k else 0
    if out is None:
        out = torch.empty((*x.shape[:-1], n), dtype=out_dtype or dtype, device=x.device)
    elif not out.is_contiguous() or out.numel() != m * n:
        raise ValueError("linear: out must be contiguous with matching size")
    if aux is not None and (aux.dtype != out.dtype or not aux.is_contiguous()):
        raise ValueError("linear: aux must be contiguous in the output dtype")
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    nh.call("xfh_linear", nh.ptr(x_c), k, nh.ptr(weight), nh.ptr(b), m, k, n, nh.dtype_code(dtype),
            nh.ptr(out), n, nh.dtype_code(out.dtype), epilogue, nh.ptr(aux), n, aux_rows,
            nh.stream_of(x.device))
    return out


def linear_batched(x: torch.Tensor, weights: torch.Tensor, bias: Optional[torch.Tensor],
                   dtype: torch.dtype, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``out[b] = x @ weights[b]^T + bias[b]`` in one launch: x [m, k] shared by every b (or
    [B, m, k]), weights [B, n, k] already in the compute dtype, bias [B, n] (fp32) or None;
    returns [B, m, n]."""
    nb, n, k = weights.shape
    if x.shape[-1] != k or not weights.is_contiguous():
        raise ValueError("linear_batched: weights must be a contiguous [B, n, k] matching x")
    shared = x.dim() == 2
    if not shared and (x.dim() != 3 or x.shape[0] != nb):
        raise ValueError("linear_batched: x must be [m, k] or [B, m, k]")
    x_c = as_dtype(x, dtype)
    m = x_c.shape[-2]
    out = torch.empty((nb, m, n), dtype=out_dtype or dtype, device=x.device)
    b = None
    if bias is not None:
        if tuple(bias.shape) != (nb, n):
            raise ValueError("linear_batched: bias must be [B, n]")
        b = bias.detach().to(torch.float32).contiguous()
    nh.call("xfh_linear_batched", nh.ptr(x_c), k, 0 if shared else m * k, nh.ptr(weights), n * k,
            nh.ptr(b), n, m, k, n, nb, nh.dtype_code(dtype), nh.ptr(out), n, m * n,
            nh.dtype_code(out.dtype), nh.stream_of(x.device))
    return out


def gated_linear_unit(x: torch.Tensor, packed: torch.Tensor, f: int, dtype: torch.dtype,
                      out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """silu(x @ Wg) * (x @ Wv) from the packed weight (``xfold/fastnn/gated_linear_unit.py:103-107``)."""
    k = x.shape[-1]
    x_c = as_dtype(x, dtype)
    m = x_c.numel() // k if k else 0
    y = torch.empty((*x.shape[:-1], f), dtype=out_dtype or dtype, device=x.device)
    nh.call("xfh_gated_linear_unit", nh.ptr(x_c), nh.ptr(packed), m, k, f, nh.dtype_code(dtype),
            nh.ptr(y), nh.dtype_code(y.dtype), nh.stream_of(x.device))
    return y


class PackedBias:
    """One [H, Q, align64(K)] block of a packed bias, passed to :func:`attention` as its
    bias (the pipelined kernel reads it as it stands): fp32 times log2(e)
    (:func:`attention_bias_pack`, :func:`pair_attention_bias` in fp32) or bf16 in natural
    units (:func:`pair_attention_bias` in bf16)."""

    def __init__(self, tensor: torch.Tensor):
        if tensor.dim() != 3 or tensor.dtype not in (torch.float32, torch.bfloat16) or not tensor.is_contiguous():
            raise ValueError("PackedBias wraps one contiguous fp32/bf16 [H, Q, align64(K)] block")
        self.tensor = tensor

    @property
    def code(self) -> int:
        return nh.BIAS_PACKED if self.tensor.dtype == torch.float32 else nh.BIAS_PACKED_BF16


def attention_bias_pack(bias: torch.Tensor) -> torch.Tensor:
    """[G, H, Q, K] biases (fp32/bf16, any strides) -> [G, H, Q, align64(K)] fp32 in the
    pipelined attention kernel's layout (times log2(e), zero pad), converted once for G calls."""
    G, H, Q, K = bias.shape
    if bias.dtype not in (torch.float32, torch.bfloat16):
        bias = bias.to(torch.float32)
    npad = (K + 63) // 64 * 64
    out = torch.empty((G, H, Q, npad), dtype=torch.float32, device=bias.device)
    shape = (ctypes.c_int64 * 4)(G, H, Q, K)
    strides = (ctypes.c_int64 * 4)(*bias.stride())
    nh.call("xfh_attention_bias_pack", nh.ptr(bias), nh.dtype_code(bias.dtype), shape, strides, nh.ptr(out),
            nh.stream_of(bias.device))
    return out


def pair_attention_bias(pair: torch.Tensor, ln_w: Optional[torch.Tensor], ln_b: Optional[torch.Tensor],
                        eps: float, weight: torch.Tensor, owner: Optional[torch.nn.Module] = None,
                        out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Linear(LayerNorm(pair)) as attention biases, [heads, N, align64(N)] in the packed
    layout (one :class:`PackedBias` per block of heads): fp32 times log2(e) (the modules'
    choice: unrounded logits), or bf16 logits (the dtype of the reference's autocast Linear
    output, half the bytes); weight [heads, 128] bf16."""
    n = pair.shape[0]
    if pair.dim() != 3 or pair.shape[1] != n or weight.dtype != torch.bfloat16:
        raise ValueError("pair_attention_bias: pair [N, N, C] and a bf16 weight")
    pair_c = pair.contiguous()
    heads = weight.shape[0]
    out = torch.empty((heads, n, (n + 63) // 64 * 64), dtype=out_dtype, device=pair.device)
    w = _fp32(ln_w, owner, "ln_weight")
    b = _fp32(ln_b, owner, "ln_bias")
    nh.call("xfh_pair_attention_bias", nh.ptr(pair_c), nh.dtype_code(pair.dtype), n, pair.shape[2],
            nh.ptr(w), nh.ptr(b), float(eps), nh.ptr(weight.contiguous()), nh.BF16, heads, nh.ptr(out),
            nh.dtype_code(out_dtype), nh.stream_of(pair.device))
    return out


class AttentionOperands:
    """Buffers of one self-attention call in the pipelined attention kernel's own layouts
    (``xfh_attention_operands_size``), for B samples of T tokens and H heads of Dh: q
    [B, H, T, Dp], k [B, H, Tpad, Dp], v^T [B, H, Dp, Tpad] (zero-initialised: the projection
    never writes their padding, so one set serves every call of that shape), the gate
    [B, T, H*Dh] and the kept-key words of the current mask."""

    def __init__(self, B: int, T: int, H: int, Dh: int, device: torch.device):
        sizes = (ctypes.c_int64 * 5)()
        nh.call("xfh_attention_operands_size", B, T, H, Dh, sizes)
        self.shape = (B, T, H, Dh)
        self.device = torch.device(device)
        self.dp, self.tpad = int(sizes[0]), int(sizes[1])
        self.q = torch.zeros(int(sizes[2]), dtype=torch.bfloat16, device=device)
        self.k = torch.zeros(int(sizes[3]), dtype=torch.bfloat16, device=device)
        self.vt = torch.zeros(int(sizes[4]), dtype=torch.bfloat16, device=device)
        self.gate = torch.empty((B, T, H * Dh), dtype=torch.bfloat16, device=device)
        self.words = torch.empty(B * (self.tpad // 64), dtype=torch.int64, device=device)
        self.words_shared = True
        self._mask_key = ()
        self._mask_ref = None

    @staticmethod
    def supported(T: int, H: int, Dh: int) -> bool:
        return Dh % 4 == 0 and 0 < Dh <= 64 and 0 < T and (T + 63) // 64 * 64 <= nh.attention_max_keys()

    def matches(self, B: int, T: int, H: int, Dh: int, device: torch.device) -> bool:
        return self.shape == (B, T, H, Dh) and self.device == torch.device(device)

    def set_mask(self, mask: Optional[torch.Tensor]) -> None:
        """Kept-key words of a key mask: None, [T] (shared by the samples) or [B, T]."""
        # Inference tensors carry no version counter: their words are recomputed every time.
        # The mask of the cached words is held, so its address cannot pass to another tensor.
        key = (None,) if mask is None else \
            None if mask.is_inference() else (id(mask), mask.data_ptr(), mask._version, tuple(mask.shape), mask.dtype)
        if key is not None and key == self._mask_key:
            return
        B, T = self.shape[0], self.shape[1]
        rows, code, m = 1, nh.BOOL, None
        if mask is not None:
            if mask.dim() == 2 and tuple(mask.shape) == (B, T):
                rows = B
            elif tuple(mask.shape) != (T,):
                raise ValueError(f"attention operands: mask must be [{T}] or [{B}, {T}]")
            m = mask if mask.dtype in (torch.bool, torch.uint8, torch.float32, torch.bfloat16) else mask.to(torch.bool)
            m = m.contiguous()
            code = nh.BOOL if m.dtype in (torch.bool, torch.uint8) else nh.dtype_code(m.dtype)
        nh.call("xfh_attention_mask_words", nh.ptr(m), code, T, rows, T, nh.ptr(self.words),
                nh.stream_of(self.device))
        self.words_shared = rows == 1
        self._mask_key = key
        self._mask_ref = mask


_SHARED_OPERANDS: "collections.OrderedDict" = collections.OrderedDict()
_SHARED_OPERANDS_MAX = 8
_SHARED_OPERANDS_LOCK = threading.Lock()


def shared_attention_operands(B: int, T: int, H: int, Dh: int, device: torch.device) -> AttentionOperands:
    """One :class:`AttentionOperands` set per (shape, device, current stream, thread), kept
    between calls: work queued on one stream runs in order, so every attention call of that
    stream can reuse the same buffers (zeroed once, padding never written) instead of
    allocating and zero-filling its own. The least recently used of more than 8 sets is
    released (the caching allocator keeps it from reuse until the queued work is done)."""
    device = torch.device(device)
    key = (B, T, H, Dh, device, nh.stream_of(device), threading.get_ident())
    with _SHARED_OPERANDS_LOCK:                  # one table for every host thread
        ops_ = _SHARED_OPERANDS.pop(key, None)
        if ops_ is None:
            ops_ = AttentionOperands(B, T, H, Dh, device)
        _SHARED_OPERANDS[key] = ops_             # (re)inserted as the most recent
        while len(_SHARED_OPERANDS) > _SHARED_OPERANDS_MAX:
            _SHARED_OPERANDS.popitem(last=False)
    return ops_


def attention_project(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                      operands: AttentionOperands, qscale: float) -> None:
    """[q | k | v | gate] = x @ weight^T + bias straight into ``operands`` (one GEMM); x
    [B*T, K] (or [B, T, K]) bf16, weight [4*H*Dh, K] bf16, bias fp32 [4*H*Dh] or None."""
    B, T, H, Dh = operands.shape
    k_dim = x.shape[-1]
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or tuple(weight.shape) != (4 * H * Dh, k_dim):
        raise ValueError("attention_project: bf16 x and a [4*H*Dh, K] bf16 weight")
    x_c = x.contiguous()
    if x_c.numel() != B * T * k_dim:
        raise ValueError("attention_project: x must hold B*T rows")
    b = None if bias is None else bias.detach().to(torch.float32).contiguous()
    nh.call("xfh_attention_project", nh.ptr(x_c), k_dim, nh.ptr(weight.contiguous()), nh.ptr(b), B, T, k_dim, H, Dh,
            float(qscale), nh.ptr(operands.q), nh.ptr(operands.k), nh.ptr(operands.vt), nh.ptr(operands.gate),
            nh.stream_of(x.device))


def attention_on_operands(operands: AttentionOperands, bias: PackedBias, out: torch.Tensor) -> torch.Tensor:
    """out [B, T, H*Dh] bf16 = sigmoid(gate) * attention over ``operands`` with a packed bias."""
    B, T, H, Dh = operands.shape
    if not isinstance(bias, PackedBias) or tuple(bias.tensor.shape) != (H, T, operands.tpad):
        raise ValueError("attention_on_operands: bias must be a packed [H, T, align64(T)] block")
    if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != B * T * H * Dh:
        raise ValueError("attention_on_operands: out must be a contiguous bf16 [B, T, H*Dh]")
    nh.call("xfh_attention_operands", nh.ptr(operands.q), nh.ptr(operands.k), nh.ptr(operands.vt),
            nh.ptr(operands.words), int(operands.words_shared), nh.ptr(bias.tensor), bias.code,
            nh.ptr(operands.gate), nh.ptr(out), B, T, H, Dh, nh.stream_of(out.device))
    return out


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
              bias: Optional[torch.Tensor], out: Optional[torch.Tensor] = None,
              scale: Optional[float] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """4-D [B, H, N, D] strided q/k/v (last dim contiguous); mask/bias broadcast to
    [B, H, Q, K] per ``xfold/fastnn/attention.py:45-66`` (bias may also be a
    :class:`PackedBias`, shared by the batch)."""
    B, H, Q, D = q.shape
    K, Dv = k.shape[2], v.shape[3]
    if k.shape[:2] != (B, H) or v.shape[:3] != (B, H, K) or k.shape[3] != D:
        raise ValueError("attention: q/k/v shapes do not match")
    dtype = q.dtype
    if k.dtype != dtype or v.dtype != dtype:
        raise ValueError("attention: q/k/v dtypes must match")
    tensors = []
    for t in (q, k, v):
        if t.stride(-1) != 1:
            t = t.contiguous()
        tensors.append(t)
    q, k, v = tensors
    if out is None:
        out = torch.empty((B, H, Q, Dv), dtype=out_dtype or dtype, device=q.device)
    if out.stride(-1) != 1:
        raise ValueError("attention: out's last dim must be contiguous")
    mask_t, mask_code = None, nh.BOOL
    mask_strides = (0, 0, 0, 0)
    if mask is not None:
        if mask.dim() == 1:
            mask = mask[None, None, None, :]
        elif mask.dim() == 2:
            mask = mask[:, None, None, :]
        # The kernels read float masks as the reference's .to(bool) does (nonzero, NaN
        # included, keeps the key: attention.py:57-61), so no conversion is launched.
        if mask.dtype not in (torch.bool, torch.uint8, torch.float32, torch.bfloat16):
            mask = mask.to(torch.bool)
        mask_t = mask.expand(B, H, Q, K)
        mask_code = nh.BOOL if mask.dtype in (torch.bool, torch.uint8) else nh.dtype_code(mask.dtype)
        mask_strides = tuple(mask_t.stride())
    bias_t, bias_code, bias_strides = None, nh.F32, (0, 0, 0, 0)
    if isinstance(bias, PackedBias):
        if tuple(bias.tensor.shape) != (H, Q, (K + 63) // 64 * 64):
            raise ValueError("attention: packed bias does not match [H, Q, align64(K)]")
        bias_t, bias_code = bias.tensor, bias.code
    elif bias is not None:
        if bias.dtype not in (torch.float32, torch.bfloat16):
            bias = bias.to(torch.float32)
        bias_t = bias.expand(B, H, Q, K)
        bias_code = nh.dtype_code(bias.dtype)
        bias_strides = tuple(bias_t.stride())
    shape = (ctypes.c_int64 * 6)(B, H, Q, K, D, Dv)
    strides = (ctypes.c_int64 * 20)(
        q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
        v.stride(0), v.stride(1), v.stride(2), out.stride(0), out.stride(1), out.stride(2),
        *mask_strides, *bias_strides)
    lib = nh.load_library()
    ws = nh.workspace(lib.xfh_dot_product_attention_workspace_size(shape, nh.dtype_code(dtype)), q.device)
    nh.call("xfh_dot_product_attention", nh.ptr(q), nh.ptr(k), nh.ptr(v), nh.dtype_code(dtype),
            nh.ptr(mask_t), mask_code, nh.ptr(bias_t), bias_code, nh.ptr(out), nh.dtype_code(out.dtype),
            shape, strides,
            float(D ** -0.5 if scale is None else scale), nh.ptr(ws), ws.numel(), nh.stream_of(q.device))
    return out
