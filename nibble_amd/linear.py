"""``QuantizedLinear`` (alias ``Int4Linear``): an inference-only linear layer
that keeps packed INT4 weights and runs them through the HIP kernels.

Mirrors reference ``w4a16/linear.py`` (constructor checks, buffers
``packed_weights`` / ``scales`` / ``bias`` in the state dict, ``from_float``,
``empty``, ``forward`` routing). Routing of ``forward``:

* CPU tensors: the pure-PyTorch ``linear_reference``;
* GPU tensors, ``fused`` and M <= ``FUSED_MAX_ROWS``: ``w4a16::linear``
  (the gfx950 GEMV / small-batch kernels);
* GPU tensors, ``fused``, group_size 128 and M <= ``NATIVE_GEMM_MAX_ROWS``
  (prompts): ``w4a16::linear`` as well, which runs the W4A16 MFMA GEMM (at
  9..16 rows of long rows, its 16-row paired form) on weights decoded in
  registers, bit-identical to the dequantized fp16 weights, with fp32
  accumulation; the reference sends these rows to dequantize + cuBLAS, and
  the result agrees with that path within its own prefill tolerance
  (reference tests/test_linear.py:207-225, rtol = atol = 1e-3);
* GPU tensors otherwise (longer prompts, ``fused=False``):
  ``w4a16::dequantize`` then ``F.linear`` (hipBLASLt) when group_size is a
  multiple of 32, else ``w4a16::linear``'s generic kernel (any M, any even
  group size).

GPU tensors never take a torch or CPU fallback: without the extension they
raise ``RuntimeError``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from nibble_amd.cuda import dequantize_cuda, linear_cuda
from nibble_amd.quantization import quantize_and_pack_weights
from nibble_amd.reference import dequantize_weights, linear_reference

# Largest M routed to the fused kernels; larger M dequantizes and uses a GEMM.
FUSED_MAX_ROWS = 8
# Largest M routed to the W4A16 GEMM when fused (group size 128): measured
# against dequantize + hipBLASLt on the 1.1B / 8B / 70B layers (e.g. M = 256,
# K 4096 x N 14336: 45 us against 81 us; M = 64, 5632 x 2048: 10 us against
# 32 us; M = 512: 69 against 95 us, 14336 x 4096 86 against 117, 8192 x 28672
# 264 against 331, and every other swept layer faster too); from M = 1024
# dequantize + hipBLASLt wins on the wide layers (4096 x 14336 138 against
# 131 us, 2048 x 11264 75 against 69) and on most layers at M = 2048, so
# longer prompts keep it.
NATIVE_GEMM_MAX_ROWS = 512


class QuantizedLinear(torch.nn.Module):
    """Inference-only linear layer backed by packed INT4 weights."""

    def __init__(
        self,
        packed_weights: torch.Tensor,
        scales: torch.Tensor,
        group_size: int = 128,
        bias: torch.Tensor | None = None,
        fused: bool = True,
    ) -> None:
        super().__init__()
        if packed_weights.dtype != torch.uint8 or packed_weights.ndim != 2:
            raise ValueError("packed_weights must be uint8 with shape [N, K / 2]")
        if scales.dtype != torch.float16 or scales.ndim != 2:
            raise ValueError("scales must be float16 with shape [N, K / group_size]")
        if packed_weights.device != scales.device:
            raise ValueError("packed_weights and scales must share a device")
        if group_size <= 0:
            raise ValueError("group_size must be greater than zero")

        self.out_features = packed_weights.shape[0]
        self.in_features = packed_weights.shape[1] * 2
        self.group_size = group_size
        if self.in_features % group_size != 0:
            raise ValueError("K must be divisible by group_size")
        expected = (self.out_features, self.in_features // group_size)
        if tuple(scales.shape) != expected:
            raise ValueError(f"scales must have shape {expected}")
        if bias is not None:
            if bias.dtype != torch.float16 or tuple(bias.shape) != (self.out_features,):
                raise ValueError("bias must be float16 with shape [N]")
            if bias.device != packed_weights.device:
                raise ValueError("bias and packed_weights must share a device")

        self.register_buffer("packed_weights", packed_weights.detach())
        self.register_buffer("scales", scales.detach())
        self.register_buffer("bias", None if bias is None else bias.detach())
        self.fused = fused
        # prompt rows up to this count take the W4A16 GEMM when fused (set it
        # to FUSED_MAX_ROWS for the reference's routing: dequantize + GEMM for
        # every M > 8)
        self.native_max_rows = NATIVE_GEMM_MAX_ROWS

    @classmethod
    def from_float(cls, layer: torch.nn.Linear, group_size: int = 128, fused: bool = True) -> "QuantizedLinear":
        """Quantize an ``nn.Linear`` (reference ``w4a16/linear.py:58-83``)."""
        if not isinstance(layer, torch.nn.Linear):
            raise TypeError("layer must be an instance of torch.nn.Linear")
        packed, scales = quantize_and_pack_weights(layer.weight.detach(), group_size)
        bias = None if layer.bias is None else layer.bias.detach().to(torch.float16)
        return cls(packed, scales, group_size=group_size, bias=bias, fused=fused)

    @classmethod
    def empty(
        cls,
        out_features: int,
        in_features: int,
        group_size: int = 128,
        bias: bool = False,
        fused: bool = True,
        device: torch.device | str | None = None,
    ) -> "QuantizedLinear":
        """Uninitialised packed storage of the right shapes (reference ``w4a16/linear.py:85-130``)."""
        if out_features <= 0 or in_features <= 0:
            raise ValueError("out_features and in_features must be greater than zero")
        if in_features % 2 != 0:
            raise ValueError("in_features must be even")
        if group_size <= 0:
            raise ValueError("group_size must be greater than zero")
        if in_features % group_size != 0:
            raise ValueError("K must be divisible by group_size")
        device = torch.device("cpu") if device is None else device
        packed = torch.empty((out_features, in_features // 2), dtype=torch.uint8, device=device)
        scales = torch.empty((out_features, in_features // group_size), dtype=torch.float16, device=device)
        bias_tensor = torch.empty((out_features,), dtype=torch.float16, device=device) if bias else None
        return cls(packed, scales, group_size=group_size, bias=bias_tensor, fused=fused)

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"group_size={self.group_size}, bias={self.bias is not None}, fused={self.fused}"
        )

    def _dequant_linear(self, activations: torch.Tensor) -> torch.Tensor:
        """fp16 weight matrix from the packed codes, then a dense GEMM."""
        if self.packed_weights.is_cuda:
            weight = dequantize_cuda(self.packed_weights, self.scales, self.group_size)
        else:
            weight = dequantize_weights(self.packed_weights, self.scales, self.group_size).to(torch.float16)
        return F.linear(activations, weight)

    def forward(self, activations: torch.Tensor) -> torch.Tensor:
        if activations.ndim < 1:
            raise ValueError("activations must have at least one dimension")
        if activations.shape[-1] != self.in_features:
            raise ValueError("activations last dimension must equal in_features")
        if activations.dtype != torch.float16:
            raise TypeError("activations must have dtype torch.float16")
        if activations.requires_grad:
            raise RuntimeError("activations must not require grad")
        if activations.device != self.packed_weights.device:
            raise ValueError("activations and packed_weights must share a device")

        output_shape = (*activations.shape[:-1], self.out_features)
        # The kernels need a dense [M, K] matrix; views from attention reshapes are copied.
        flat = activations.contiguous().reshape(-1, self.in_features)
        rows = flat.shape[0]
        if flat.is_cuda:
            if not self.packed_weights.is_contiguous():
                raise ValueError("packed_weights must be contiguous")
            if not self.scales.is_contiguous():
                raise ValueError("scales must be contiguous")
            if self.fused and rows <= FUSED_MAX_ROWS:
                out = linear_cuda(flat, self.packed_weights, self.scales, self.group_size)
            elif self.fused and self.group_size == 128 and rows <= self.native_max_rows:
                out = linear_cuda(flat, self.packed_weights, self.scales, self.group_size)
            elif self.group_size % 32 == 0:
                out = self._dequant_linear(flat)
            else:
                out = linear_cuda(flat, self.packed_weights, self.scales, self.group_size)
        else:
            out = linear_reference(flat, self.packed_weights, self.scales, self.group_size)
        out = out.reshape(output_shape)
        if self.bias is not None:
            out = out + self.bias
        return out


# The name the W4A16 API documentation uses for the same class.
Int4Linear = QuantizedLinear
