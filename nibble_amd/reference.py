"""Pure-PyTorch W4A16 arithmetic: the path ``QuantizedLinear`` takes for CPU
tensors, and the exact dequantization the HIP kernels are specified by.

Mirrors the public functions of reference ``w4a16/reference.py`` (same names,
arguments, checks and results). On GPU tensors these functions run torch's
own GPU ops; the product's GPU path uses the HIP kernels instead
(``nibble_amd.cuda``).
"""

from __future__ import annotations

import torch

from nibble_amd.quantization import unpack_int4


def dequantize_weights(
    packed_weights: torch.Tensor, scales: torch.Tensor, group_size: int = 128
) -> torch.Tensor:
    """Exact fp32 weights ``code * fp32(scale)`` [N, K].

    Follows reference ``w4a16/reference.py:6-46``. The product of a 4-bit
    code and an fp16 scale has at most 15 significant bits, so it is exact in
    fp32; ``.to(torch.float16)`` of it is the bit pattern the HIP dequantize
    kernel must reproduce.
    """
    if packed_weights.dtype != torch.uint8:
        raise TypeError("packed_weights must have dtype torch.uint8")
    if scales.dtype != torch.float16:
        raise TypeError("scales must have dtype torch.float16")
    if packed_weights.ndim != 2:
        raise ValueError("packed_weights must have shape [N, K / 2]")
    if scales.ndim != 2:
        raise ValueError("scales must have shape [N, K / group_size]")
    if packed_weights.device != scales.device:
        raise ValueError("packed_weights and scales must be on the same device")
    if group_size <= 0:
        raise ValueError("group_size must be greater than zero")

    codes = unpack_int4(packed_weights)
    rows, cols = codes.shape
    if cols % group_size != 0:
        raise ValueError("K must be divisible by group_size")
    expected = (rows, cols // group_size)
    if tuple(scales.shape) != expected:
        raise ValueError(f"scales must have shape {expected}, got {tuple(scales.shape)}")

    grouped = codes.to(torch.float32).reshape(rows, cols // group_size, group_size)
    return (grouped * scales.to(torch.float32).unsqueeze(2)).reshape(rows, cols)


def linear_reference(
    activations: torch.Tensor,
    packed_weights: torch.Tensor,
    scales: torch.Tensor,
    group_size: int = 128,
) -> torch.Tensor:
    """``fp16(fp32(x) @ W^T)`` with W from :func:`dequantize_weights`.

    Follows reference ``w4a16/reference.py:49-80``.
    """
    if activations.dtype != torch.float16:
        raise TypeError("activations must have dtype torch.float16")
    if activations.ndim != 2:
        raise ValueError("activations must have shape [M, K]")
    if activations.device != packed_weights.device or activations.device != scales.device:
        raise ValueError("activations, packed_weights, and scales must share a device")

    weight = dequantize_weights(packed_weights, scales, group_size)
    if activations.shape[1] != weight.shape[1]:
        raise ValueError("activations and weights must have the same K dimension")
    return torch.matmul(activations.to(torch.float32), weight.t()).to(torch.float16)
