"""Model patching: swap ``nn.Linear`` children for ``QuantizedLinear`` and
load packed state dicts without materialising fp16 weights.

Mirrors reference ``w4a16/integration.py`` (same functions, arguments,
warnings and return values).
"""

from __future__ import annotations

import warnings

import torch

from nibble_amd.linear import QuantizedLinear


def replace_linear_layers(
    module: torch.nn.Module,
    group_size: int = 128,
    prefix: str = "",
    fused: bool = True,
    packed_only: bool = False,
) -> int:
    """Recursively replace compatible ``nn.Linear`` children; returns the count.

    Layers whose ``in_features`` is not a multiple of ``group_size`` are kept
    and reported with a ``UserWarning`` naming their qualified path.
    ``packed_only=True`` allocates empty packed storage from the layer shape
    without reading the source weights (for a later ``load_state_dict``).
    Follows reference ``w4a16/integration.py:8-69``.
    """
    if group_size <= 0:
        raise ValueError("group_size must be greater than zero")

    count = 0
    for name, child in list(module.named_children()):
        qualified = f"{prefix}.{name}" if prefix else name
        if isinstance(child, QuantizedLinear):
            continue
        if not isinstance(child, torch.nn.Linear):
            count += replace_linear_layers(child, group_size, prefix=qualified, fused=fused, packed_only=packed_only)
            continue
        if child.in_features % group_size != 0:
            warnings.warn(
                f"Skipping linear layer '{qualified}' because in_features={child.in_features} "
                f"is not divisible by group_size={group_size}",
                UserWarning,
                stacklevel=2,
            )
            continue
        if packed_only:
            replacement = QuantizedLinear.empty(
                out_features=child.out_features,
                in_features=child.in_features,
                group_size=group_size,
                bias=child.bias is not None,
                fused=fused,
                device=child.weight.device,
            )
        else:
            replacement = QuantizedLinear.from_float(child, group_size=group_size, fused=fused)
        replacement.train(child.training)
        setattr(module, name, replacement)
        count += 1
    return count


def _restore_computed_buffers(module: torch.nn.Module) -> None:
    """Recompute non-persistent buffers that ``to_empty`` left uninitialised.

    HuggingFace rotary-embedding modules keep ``inv_freq`` (and
    ``original_inv_freq``) as non-persistent buffers; they are recomputed from
    the module's config. Follows reference ``w4a16/integration.py:72-94``.
    """
    for child in module.modules():
        compute = getattr(child, "compute_default_rope_parameters", None)
        if compute is None or not hasattr(child, "config"):
            continue
        inv_freq = getattr(child, "inv_freq", None)
        if inv_freq is None:
            continue
        values, attention_scaling = compute(child.config)
        inv_freq.copy_(values.to(device=inv_freq.device, dtype=inv_freq.dtype))
        original = getattr(child, "original_inv_freq", None)
        if original is not None:
            original.copy_(values.to(device=original.device, dtype=original.dtype))
        child.attention_scaling = attention_scaling


def load_packed_state_dict(
    module: torch.nn.Module,
    state_dict: dict,
    group_size: int = 128,
    device: str | torch.device = "cpu",
    fused: bool = True,
) -> int:
    """Patch ``module`` (which may live on the meta device) with empty packed
    layers, allocate everything on ``device`` and load ``state_dict``.

    Follows reference ``w4a16/integration.py:97-119``.
    """
    count = replace_linear_layers(module, group_size=group_size, fused=fused, packed_only=True)
    module.to_empty(device=device)
    module.load_state_dict(state_dict)
    _restore_computed_buffers(module)
    return count
