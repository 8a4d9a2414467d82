"""Quantisation of BitNet b1.58 (same API as bitnet-tt's
``src/bitnet_tt/utils/quantization.py``).

* weights: ternary {-1, 0, +1} by absmean, ``s = max(mean|W|, eps)``,
  ``q = clip(round_half_even(W / s), -1, 1)`` (quantization.py:15-57);
* activations: 8-bit per-token absmax, ``a = max(max|x|, eps)``,
  ``scale = 127 / a``, ``q = clip(round_half_even(x * scale), -128, 127)``
  (quantization.py:60-91).

numpy arrays take the host path the reference takes (load-time use, the same
numpy calls, so scales agree to the bit).  Tensors on a ROCm device run the
gfx950 kernels of libbtl.so, which reproduce the same values: the weight scale
follows numpy's float32 summation order and the activation quantiser rounds
exactly as above.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray


def _is_device_tensor(x) -> bool:
    try:
        import torch
    except ImportError:  # pragma: no cover
        return False
    return isinstance(x, torch.Tensor) and x.is_cuda


def compute_weight_scale(weight, eps: float = 1e-5):
    """``max(mean(|W|), eps)`` (quantization.py:15-29)."""
    if _is_device_tensor(weight):
        return weight_quant_ternary(weight, eps)[1]
    scale = np.mean(np.abs(weight))
    return np.maximum(scale, eps)


def weight_quant_ternary(weight, eps: float = 1e-5):
    """Absmean ternary quantisation (quantization.py:32-57).

    numpy in -> (int8 array, numpy float32 scale).  A float32 ROCm tensor in ->
    (int8 tensor, python float scale) computed by ``btl_weight_quant_ternary``.
    """
    if _is_device_tensor(weight):
        return _weight_quant_device(weight, eps)
    scale = compute_weight_scale(weight, eps)
    weight_scaled = weight / scale
    weight_quant = np.clip(np.round(weight_scaled), -1, 1).astype(np.int8)
    return weight_quant, scale


def _weight_quant_device(weight, eps: float):
    import torch

    from .. import _native as N

    if weight.dtype != torch.float32:
        raise ValueError("device weight quantisation expects a float32 tensor")
    N.require_cuda(weight, "weight")
    n = weight.numel()
    q = torch.empty(weight.shape, dtype=torch.int8, device=weight.device)
    scale = torch.empty(1, dtype=torch.float32, device=weight.device)
    scratch_bytes = int(N.lib().btl_weight_quant_scratch_bytes(n))
    scratch = torch.empty(max(scratch_bytes, 4), dtype=torch.uint8, device=weight.device)
    N.check(
        N.lib().btl_weight_quant_ternary(
            N.ptr(weight), n, eps, N.ptr(q), N.ptr(scale), N.ptr(scratch), scratch.numel(),
            N.stream_of(weight.device),
        ),
        "btl_weight_quant_ternary",
    )
    return q, float(scale.item())


def activation_quant_absmax(x, num_bits: int = 8, eps: float = 1e-5):
    """Per-token absmax quantisation (quantization.py:60-91).

    numpy in -> (int8 array, scale array with keepdims).  A bf16 ROCm tensor
    [..., K] in -> (int8 tensor [..., K], float32 scale tensor [..., 1]) from
    ``btl_quant_absmax`` (8 bits only, K a multiple of 32).
    """
    if _is_device_tensor(x):
        if num_bits != 8 or eps != 1e-5:
            raise ValueError("the device quantiser implements the 8-bit, eps=1e-5 case")
        return _act_quant_device(x)
    q_b = 2 ** (num_bits - 1) - 1
    x_abs_max = np.max(np.abs(x), axis=-1, keepdims=True)
    x_abs_max = np.maximum(x_abs_max, eps)
    scale = q_b / x_abs_max
    x_quant = np.clip(np.round(x * scale), -q_b - 1, q_b).astype(np.int8)
    return x_quant, scale


def _act_quant_device(x):
    import torch

    from .. import _native as N

    if x.dtype != torch.bfloat16:
        raise ValueError("device activation quantisation expects a bfloat16 tensor")
    N.require_cuda(x, "x")
    k = x.shape[-1]
    m = x.numel() // k
    dev = x.device
    L = N.lib()
    rows = 32 * ((m + 31) // 32)
    xa = torch.empty(int(L.btl_act_bytes(m, k)), dtype=torch.uint8, device=dev)
    a_dq = torch.empty(rows, dtype=torch.float32, device=dev)
    rowsum = torch.empty(rows, dtype=torch.int32, device=dev)
    scale = torch.empty(m, dtype=torch.float32, device=dev)
    q = torch.empty(x.shape, dtype=torch.int8, device=dev)
    N.check(
        L.btl_quant_absmax(N.ptr(x), m, k, k, None, 0.0, N.ptr(xa), N.ptr(a_dq), N.ptr(rowsum), N.ptr(scale),
                           N.ptr(q), None, N.stream_of(dev)),
        "btl_quant_absmax",
    )
    return q, scale.reshape(x.shape[:-1] + (1,))


def dequantize_weight(weight_quant: NDArray[np.int8], scale) -> NDArray[np.floating]:
    """``q * scale`` in float32 (quantization.py:94-108)."""
    return weight_quant.astype(np.float32) * float(scale)


def pack_ternary_weights(weight_quant: NDArray[np.int8]) -> NDArray[np.uint8]:
    """Flat offset-coded packing used for analysis: -1 -> 0b00, 0 -> 0b01,
    +1 -> 0b10, four per byte, first in the top bits, padded with 0b01
    (quantization.py:111-138)."""
    flat = (np.asarray(weight_quant).astype(np.int32) + 1).reshape(-1)
    pad = (4 - flat.size % 4) % 4
    if pad:
        flat = np.pad(flat, (0, pad), constant_values=1)
    f = flat.reshape(-1, 4)
    return ((f[:, 0] << 6) | (f[:, 1] << 4) | (f[:, 2] << 2) | f[:, 3]).astype(np.uint8)


def unpack_ternary_weights(packed: NDArray[np.uint8], original_shape: tuple[int, ...]) -> NDArray[np.int8]:
    """Inverse of :func:`pack_ternary_weights` (quantization.py:141-174)."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1, 1)
    vals = ((p >> np.array([6, 4, 2, 0], dtype=np.uint8)) & 0x03).reshape(-1).astype(np.int8) - 1
    total = int(np.prod(original_shape)) if len(original_shape) else 1
    return vals[:total].reshape(original_shape)
