"""Python wrappers of the torch ops ``w4a16::linear`` / ``w4a16::dequantize``.

Mirrors reference ``w4a16/cuda.py``: importing the compiled extension
(``nibble_amd._C``, here a thin libtorch shim over the HIP C ABI) registers
the ops; a missing extension is recorded, ``cuda_extension_available()``
reports it and the wrappers raise ``RuntimeError``. There is no fallback:
GPU tensors only ever run the HIP kernels. On PyTorch-ROCm "cuda" tensors
are HIP tensors, so the reference's names are kept.
"""

from __future__ import annotations

import importlib

import torch

try:
    importlib.import_module("nibble_amd._C")
except (ImportError, OSError) as error:
    _EXTENSION_LOAD_ERROR: Exception | None = error
else:
    _EXTENSION_LOAD_ERROR = None


if _EXTENSION_LOAD_ERROR is None:
    # Shape/dtype-only implementations so torch.compile can trace through the
    # ops with fake tensors (reference w4a16/cuda.py:14-36).
    @torch.library.register_fake("w4a16::linear")
    def _linear_fake(activations, packed_weights, scales, group_size):
        return activations.new_empty((activations.shape[0], packed_weights.shape[0]))

    @torch.library.register_fake("w4a16::dequantize")
    def _dequantize_fake(packed_weights, scales, group_size):
        return packed_weights.new_empty(
            (packed_weights.shape[0], packed_weights.shape[1] * 2), dtype=torch.float16
        )


def cuda_extension_available() -> bool:
    """Whether the compiled W4A16 HIP extension is loaded."""
    return _EXTENSION_LOAD_ERROR is None


def extension_load_error() -> Exception | None:
    return _EXTENSION_LOAD_ERROR


def _require_extension() -> None:
    if _EXTENSION_LOAD_ERROR is not None:
        raise RuntimeError(
            "The W4A16 HIP extension is not built. Build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'`."
        ) from _EXTENSION_LOAD_ERROR


def linear_cuda(
    activations: torch.Tensor,
    packed_weights: torch.Tensor,
    scales: torch.Tensor,
    group_size: int = 128,
) -> torch.Tensor:
    """Fused W4A16 linear on the GPU (reference ``w4a16/cuda.py:52-69``).

    group_size 128 with 16-byte aligned operands and M <= 8 runs the tuned
    gfx950 kernels; anything else runs the generic HIP kernel.
    """
    _require_extension()
    return torch.ops.w4a16.linear(activations, packed_weights, scales, group_size)


def dequantize_cuda(
    packed_weights: torch.Tensor,
    scales: torch.Tensor,
    group_size: int = 128,
) -> torch.Tensor:
    """Packed INT4 -> fp16 [N, K] in one pass (reference ``w4a16/cuda.py:72-83``).

    Bit-identical to ``dequantize_weights(...).to(torch.float16)``; needs
    group_size a multiple of 32 and 16-byte aligned packed weights.
    """
    _require_extension()
    return torch.ops.w4a16.dequantize(packed_weights, scales, group_size)
