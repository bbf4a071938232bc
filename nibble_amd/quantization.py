"""Packed INT4 format and the round-to-nearest group quantizer.

Format (must stay byte-identical to reference ``w4a16/quantization.py``):
weights are signed codes in [-7, 7] (the kernels also accept -8), two per
byte, the even-k code in the low nibble and the odd-k code in the high
nibble, two's complement. ``packed_weights`` is ``uint8 [N, K/2]`` and
``scales`` is ``float16 [N, K/group_size]``.

The quantizer is symmetric absmax RTN per group of ``group_size`` weights
along K: ``s = amax|w| / 7`` in fp32 (1.0 for an all-zero group), codes
``clamp(round_half_even(w / s), -7, 7)`` computed with the fp32 ``s``, and
the stored scale is ``fp16(s)``. The steps are fixed by the format: any
other order or precision would produce different packed bytes.
"""

from __future__ import annotations

import torch


def pack_int4(quantized_weights: torch.Tensor) -> torch.Tensor:
    """int8 codes [N, K] in [-7, 7] -> uint8 [N, K/2].

    Follows reference ``w4a16/quantization.py:4-28`` (same checks, same bytes).
    """
    if quantized_weights.dtype != torch.int8:
        raise TypeError("quantized_weights int4 value must have int8 dtype")
    if quantized_weights.ndim != 2:
        raise ValueError("quantized_weights shape mismatch, expected: [N,K]")
    if quantized_weights.shape[1] % 2 != 0:
        raise ValueError("K num of weights per row, must be even so two weights = 1 byte")
    if bool(((quantized_weights < -7) | (quantized_weights > 7)).any()):
        raise ValueError("quantized_weights val must be between [-7, 7]")

    # Nibbles as small non-negative integers, then one byte per (even, odd) pair.
    nibbles = quantized_weights.to(torch.int16) & 0x0F
    pairs = nibbles.reshape(quantized_weights.shape[0], -1, 2)
    return (pairs[..., 0] | (pairs[..., 1] << 4)).to(torch.uint8)


def unpack_int4(packed_weights: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K/2] -> int8 codes [N, K] in [-8, 7].

    Follows reference ``w4a16/quantization.py:31-63``.
    """
    if packed_weights.dtype != torch.uint8:
        raise TypeError("packed_weights must have uint8 dtype")
    if packed_weights.ndim != 2:
        raise ValueError("packed_weights shape mismatch, should be [N,K]")

    wide = packed_weights.to(torch.int16)
    # (v ^ 8) - 8 sign-extends a 4-bit two's-complement value.
    low = ((wide & 0x0F) ^ 8) - 8
    high = ((wide >> 4) ^ 8) - 8
    codes = torch.stack((low, high), dim=-1).reshape(packed_weights.shape[0], -1)
    return codes.to(torch.int8)


def quantize_groupwise(
    weights: torch.Tensor, group_size: int = 128
) -> tuple[torch.Tensor, torch.Tensor]:
    """fp16/fp32 weights [N, K] -> (int8 codes [N, K], fp16 scales [N, K/G]).

    Follows reference ``w4a16/quantization.py:65-102``.
    """
    if weights.dtype not in (torch.float16, torch.float32):
        raise TypeError("weights must have dtype torch.float16 or torch.float32")
    if weights.ndim != 2:
        raise ValueError("weights must have shape [N, K]")
    if group_size <= 0:
        raise ValueError("group_size must be greater than zero")
    if weights.shape[1] % group_size != 0:
        raise ValueError("K must be divisible by group_size")

    rows, cols = weights.shape
    groups = weights.to(torch.float32).reshape(rows, cols // group_size, group_size)
    amax = groups.abs().amax(dim=2, keepdim=True)
    # amax / 7 as a correctly rounded fp32 quotient on every device: torch's
    # GPU kernels divide by a Python scalar as a product with its rounded
    # reciprocal (an ulp off for about half of the quotients, which moves ~5e-5
    # of the fp16 scales), so the divisor is a tensor and GPU quantization
    # writes the same bytes as the CPU path
    scale = torch.where(amax == 0, torch.ones_like(amax), amax / torch.full_like(amax, 7.0))
    codes = torch.round(groups / scale).clamp_(-7, 7).to(torch.int8).reshape(rows, cols)
    return codes, scale.squeeze(2).to(torch.float16)


def quantize_and_pack_weights(
    weights: torch.Tensor, group_size: int = 128
) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize then pack (reference ``w4a16/quantization.py:105-113``)."""
    codes, scales = quantize_groupwise(weights, group_size)
    return pack_int4(codes), scales
