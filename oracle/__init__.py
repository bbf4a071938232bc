"""CPU oracle for the W4A16 path -- TEST INFRASTRUCTURE, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or as
the timed CPU baseline). The product package ``nibble_amd`` never imports it.

numpy front end over ``oracle/liboracle.so`` (built from ``oracle/oracle.c``
by ``oracle/Makefile``), restating the reference's arithmetic:

=========================  ==========================================
function                   reference (chris320211/Nibble)
=========================  ==========================================
``pack_int4``              ``w4a16/quantization.py:4-28``
``unpack_int4``            ``w4a16/quantization.py:31-63``
``quantize_groupwise``     ``w4a16/quantization.py:65-102``
``quantize_and_pack``      ``w4a16/quantization.py:105-113``
``dequantize_f32``         ``w4a16/reference.py:6-46``
``dequantize_f16``         ``w4a16/reference.py:6-46`` then ``.to(float16)``
``linear``                 ``w4a16/reference.py:49-80``
``f32_to_f16``             IEEE 754 binary16, round to nearest even
=========================  ==========================================

Every function is pinned by ``tests/test_oracle.py`` (known-answer vectors of
the reference's own tests in ``tests/golden/kat.json`` plus closed forms
computed independently with numpy); none is "parity unpinned".

The reference's own implementation is not built or run: its CPU path is
Python (read, not run) and its kernels are CUDA (no nvcc here), so there is
no ``oracle/_ref``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


def build() -> None:
    """Compile ``liboracle.so`` with gcc (``make -C oracle``)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_pack_int4.argtypes = [_ptr, _i64, _i64, _ptr]
    lib.oracle_pack_int4.restype = ctypes.c_int
    lib.oracle_unpack_int4.argtypes = [_ptr, _i64, _i64, _ptr]
    lib.oracle_unpack_int4.restype = None
    lib.oracle_quantize_groupwise.argtypes = [_ptr, _i64, _i64, _i64, _ptr, _ptr]
    lib.oracle_quantize_groupwise.restype = ctypes.c_int
    lib.oracle_dequantize_f32.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _ptr]
    lib.oracle_dequantize_f32.restype = None
    lib.oracle_dequantize_f16.argtypes = [_ptr, _ptr, _i64, _i64, _i64, _ptr]
    lib.oracle_dequantize_f16.restype = None
    lib.oracle_linear.argtypes = [_ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, ctypes.c_int]
    lib.oracle_linear.restype = ctypes.c_int
    _lib = lib
    return lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


def f32_to_f16(values) -> np.ndarray:
    """fp32 -> binary16 (RNE) elementwise; returns an np.float16 array."""
    lib = _load()
    v = _c(values, np.float32)
    out = np.array([lib.oracle_f32_to_f16(float(x)) for x in v.ravel()], dtype=np.uint16)
    return out.view(np.float16).reshape(v.shape)


def f16_to_f32(values) -> np.ndarray:
    lib = _load()
    v = _c(values, np.float16).view(np.uint16)
    out = np.array([lib.oracle_f16_to_f32(int(x)) for x in v.ravel()], dtype=np.float32)
    return out.reshape(v.shape)


def pack_int4(codes) -> np.ndarray:
    """int8 codes [N, K] in [-7, 7] -> uint8 [N, K/2] (even k in the low nibble)."""
    lib = _load()
    q = _c(codes, np.int8)
    if q.ndim != 2:
        raise ValueError("codes must be [N, K]")
    n, k = q.shape
    out = np.empty((n, k // 2), dtype=np.uint8)
    rc = lib.oracle_pack_int4(_p(q), n, k, _p(out))
    if rc == 1:
        raise ValueError("codes must be in [-7, 7]")
    if rc == 2:
        raise ValueError("K must be even")
    return out


def unpack_int4(packed) -> np.ndarray:
    lib = _load()
    p = _c(packed, np.uint8)
    n, kh = p.shape
    out = np.empty((n, 2 * kh), dtype=np.int8)
    lib.oracle_unpack_int4(_p(p), n, kh, _p(out))
    return out


def quantize_groupwise(weights, group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """fp32 (or fp16) weights [N, K] -> (int8 codes [N, K], float16 scales [N, K/G])."""
    lib = _load()
    w = _c(np.asarray(weights).astype(np.float32), np.float32)
    n, k = w.shape
    if group_size <= 0 or k % group_size:
        raise ValueError("K must be divisible by group_size")
    q = np.empty((n, k), dtype=np.int8)
    s = np.empty((n, k // group_size), dtype=np.uint16)
    lib.oracle_quantize_groupwise(_p(w), n, k, group_size, _p(q), _p(s))
    return q, s.view(np.float16)


def quantize_and_pack(weights, group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    q, s = quantize_groupwise(weights, group_size)
    return pack_int4(q), s


def dequantize_f32(packed, scales, group_size: int = 128) -> np.ndarray:
    lib = _load()
    p = _c(packed, np.uint8)
    s = _c(scales, np.float16).view(np.uint16)
    n, kh = p.shape
    k = 2 * kh
    out = np.empty((n, k), dtype=np.float32)
    lib.oracle_dequantize_f32(_p(p), _p(s), n, k, group_size, _p(out))
    return out


def dequantize_f16(packed, scales, group_size: int = 128) -> np.ndarray:
    lib = _load()
    p = _c(packed, np.uint8)
    s = _c(scales, np.float16).view(np.uint16)
    n, kh = p.shape
    k = 2 * kh
    out = np.empty((n, k), dtype=np.uint16)
    lib.oracle_dequantize_f16(_p(p), _p(s), n, k, group_size, _p(out))
    return out.view(np.float16)


def linear(activations, packed, scales, group_size: int = 128, threads: int = 0) -> np.ndarray:
    """fp16 [M, K] x packed INT4 [N, K/2] -> fp16 [M, N] (fp32 weights, exact-ish sum)."""
    lib = _load()
    x = _c(activations, np.float16).view(np.uint16)
    p = _c(packed, np.uint8)
    s = _c(scales, np.float16).view(np.uint16)
    m, k = x.shape
    n = p.shape[0]
    if p.shape[1] * 2 != k:
        raise ValueError("activations and weights must have the same K dimension")
    out = np.empty((m, n), dtype=np.uint16)
    rc = lib.oracle_linear(_p(x), _p(p), _p(s), m, n, k, group_size, _p(out), int(threads))
    if rc != 0:
        raise ValueError(f"oracle_linear failed with code {rc}")
    return out.view(np.float16)
