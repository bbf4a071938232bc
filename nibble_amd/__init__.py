"""MI355X-native W4A16 linear layer (gfx950 HIP kernels behind the ``w4a16`` API).

The public names are those of reference ``w4a16/__init__.py:15-28``;
``Int4Linear`` is an alias of ``QuantizedLinear``. The package is also
importable as ``w4a16`` (see the top-level ``w4a16`` package), so code
written against the reference runs unchanged.
"""

from nibble_amd.checkpoint import load_quantized_weight_checkpoint, save_quantized_weight_checkpoint
from nibble_amd.cuda import cuda_extension_available, dequantize_cuda, linear_cuda
from nibble_amd.integration import load_packed_state_dict, replace_linear_layers
from nibble_amd.linear import Int4Linear, QuantizedLinear
from nibble_amd.quantization import pack_int4, quantize_and_pack_weights, quantize_groupwise, unpack_int4

__all__ = [
    "QuantizedLinear",
    "Int4Linear",
    "pack_int4",
    "unpack_int4",
    "quantize_groupwise",
    "quantize_and_pack_weights",
    "save_quantized_weight_checkpoint",
    "load_quantized_weight_checkpoint",
    "replace_linear_layers",
    "load_packed_state_dict",
    "linear_cuda",
    "dequantize_cuda",
    "cuda_extension_available",
]
