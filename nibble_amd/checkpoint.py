"""Single-matrix packed checkpoint: a ``torch.save`` dict of
``{format, version, packed_weights, scales, group_size, original_shape}``.

The layout (keys, ``FORMAT_NAME``, ``FORMAT_VERSION``) is the reference's
(``w4a16/checkpoint.py:6-56``) so files are interchangeable; loading uses
``torch.load(weights_only=True)`` and validates everything it reads.
"""

from __future__ import annotations

from pathlib import Path

import torch

FORMAT_NAME = "w4a16-linear"
FORMAT_VERSION = 1


def _validate_quantized_tensors(packed_weights, scales, group_size) -> tuple[int, int]:
    if packed_weights.dtype != torch.uint8 or packed_weights.ndim != 2:
        raise ValueError("packed_weights must be a uint8 tensor shaped [N, K / 2]")
    if scales.dtype != torch.float16 or scales.ndim != 2:
        raise ValueError("scales must be a float16 tensor shaped [N, K / group_size]")
    if packed_weights.device != scales.device:
        raise ValueError("packed_weights and scales must share a device")
    if group_size <= 0:
        raise ValueError("group_size must be greater than zero")
    out_features = packed_weights.shape[0]
    in_features = packed_weights.shape[1] * 2
    if in_features % group_size != 0:
        raise ValueError("K must be divisible by group_size")
    expected = (out_features, in_features // group_size)
    if tuple(scales.shape) != expected:
        raise ValueError(f"scales must have shape {expected}")
    return out_features, in_features


def save_quantized_weight_checkpoint(
    path: str | Path, packed_weights: torch.Tensor, scales: torch.Tensor, group_size: int = 128
) -> None:
    """Write one packed matrix (reference ``w4a16/checkpoint.py:36-56``)."""
    shape = _validate_quantized_tensors(packed_weights, scales, group_size)
    torch.save(
        {
            "format": FORMAT_NAME,
            "version": FORMAT_VERSION,
            "packed_weights": packed_weights.detach().cpu(),
            "scales": scales.detach().cpu(),
            "group_size": group_size,
            "original_shape": shape,
        },
        Path(path),
    )


def load_quantized_weight_checkpoint(
    path: str | Path, map_location: str | torch.device = "cpu"
) -> tuple[torch.Tensor, torch.Tensor, int]:
    """Read and validate one packed matrix (reference ``w4a16/checkpoint.py:59-94``)."""
    checkpoint = torch.load(Path(path), map_location=map_location, weights_only=True)
    if not isinstance(checkpoint, dict):
        raise ValueError("checkpoint must contain a dictionary")
    if checkpoint.get("format") != FORMAT_NAME:
        raise ValueError("checkpoint has an unsupported format")
    if checkpoint.get("version") != FORMAT_VERSION:
        raise ValueError("checkpoint has an unsupported version")
    packed = checkpoint.get("packed_weights")
    scales = checkpoint.get("scales")
    group_size = checkpoint.get("group_size")
    if not isinstance(packed, torch.Tensor):
        raise ValueError("checkpoint is missing packed_weights")
    if not isinstance(scales, torch.Tensor):
        raise ValueError("checkpoint is missing scales")
    if not isinstance(group_size, int):
        raise ValueError("checkpoint is missing group_size")
    shape = _validate_quantized_tensors(packed, scales, group_size)
    if tuple(checkpoint.get("original_shape", ())) != shape:
        raise ValueError("checkpoint original_shape does not match its tensors")
    return packed, scales, group_size
