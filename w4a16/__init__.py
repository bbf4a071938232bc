"""Drop-in import name for code written against the reference's ``w4a16`` package.

``import w4a16`` / ``from w4a16.linear import QuantizedLinear`` /
``importlib.import_module("w4a16._C")`` resolve to the same module objects as
``nibble_amd`` and its submodules (one implementation, two import names).
"""

import importlib as _importlib
import sys as _sys

import nibble_amd as _impl
from nibble_amd import *  # noqa: F401,F403
from nibble_amd import __all__  # noqa: F401

for _name in ("quantization", "reference", "cuda", "linear", "integration", "checkpoint"):
    _module = _importlib.import_module(f"nibble_amd.{_name}")
    _sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module

if _impl.cuda_extension_available():
    _sys.modules[f"{__name__}._C"] = _sys.modules["nibble_amd._C"]
