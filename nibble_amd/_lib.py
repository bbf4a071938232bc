"""ctypes binding of the C ABI in ``include/w4a16_hip.h`` (``libw4a16_hip.so``).

This is the binding a non-torch caller would write; the torch ops in
``nibble_amd._C`` call the same entry points from C++. torch is imported
first so that the library binds to the HIP runtime torch already loaded
(both resolve the same ``libamdhip64.so.7`` soname).
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the process's HIP runtime before the library)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libw4a16_hip.so")

W4A16_OK = 0
W4A16_ERR_GROUP_SIZE = 1
W4A16_ERR_SHAPE = 2
W4A16_ERR_ALIGNMENT = 3
W4A16_ERR_NULL = 4
W4A16_ERR_CONFIG = 5
W4A16_ERR_LAUNCH = 6
W4A16_ERR_TOO_LARGE = 7

KERNEL_NONE = 0
KERNEL_VALU = 1
KERNEL_MFMA = 2
KERNEL_GENERIC = 3
KERNEL_DIAG = 4
KERNEL_VALU_OFFSET = 5
KERNEL_ONESHOT = 6
KERNEL_MFMA_ONESHOT = 7
KERNEL_MFMA_PAIR = 8
KERNEL_STREAM = 9
KERNEL_GEMM = 10
KERNEL_PAIR_STREAM = 11
KERNEL_GEMM_LDS = 12
KERNEL_PAIR_SPLIT = 13
KERNEL_GEMM32 = 14
KERNEL_PAIR_RING = 15
KERNEL_NAMES = {KERNEL_NONE: "none", KERNEL_VALU: "valu", KERNEL_MFMA: "mfma", KERNEL_GENERIC: "generic",
                KERNEL_DIAG: "diag", KERNEL_VALU_OFFSET: "valu_offset",
                KERNEL_ONESHOT: "oneshot", KERNEL_MFMA_ONESHOT: "mfma_oneshot",
                KERNEL_MFMA_PAIR: "mfma_pair", KERNEL_STREAM: "stream",
                KERNEL_GEMM: "gemm", KERNEL_PAIR_STREAM: "pair_stream",
                KERNEL_GEMM_LDS: "gemm_lds", KERNEL_PAIR_SPLIT: "pair_split", KERNEL_GEMM32: "gemm32",
                KERNEL_PAIR_RING: "pair_ring"}

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_ip = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); every symbol declared in include/w4a16_hip.h
SIGNATURES = {
    "w4a16_linear_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "w4a16_dequantize_f16": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "w4a16_check_linear_shapes": (ctypes.c_int, [_i64] * 7),
    "w4a16_check_dequantize_shapes": (ctypes.c_int, [_i64] * 5 + [ctypes.c_uint64]),
    "w4a16_plan_linear": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _ip, _ip, _ip, _ip, _ip]),
    "w4a16_plan_linear_ws": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, _ip, _ip, _ip, _ip, _ip]),
    "w4a16_linear_workspace_bytes": (_i64, [_i64] * 4),
    "w4a16_linear_ws_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "w4a16_linear_noalloc_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "w4a16_linear_f16_tuned": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp] + [ctypes.c_int] * 5 + [_vp, _i64],
    ),
    "w4a16_last_error": (ctypes.c_char_p, []),
    "w4a16_version": (ctypes.c_char_p, []),
}

# every symbol declared in include/w4a16_decode.h
DECODE_SIGNATURES = {
    "w4a16_gemv_fused_f16": (
        ctypes.c_int,
        [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _i64, _i64, _i64, ctypes.c_int, _vp],
    ),
    "w4a16_decode_attention_f16": (ctypes.c_int, [_vp] * 7 + [_i64] * 4 + [_vp]),
    "w4a16_decode_attention_split_f16": (ctypes.c_int, [_vp] * 7 + [_i64] * 5 + [_vp, _i64, _vp]),
    "w4a16_attention_o_f16": (ctypes.c_int, [_vp] * 8 + [_i64] * 6 + [_vp]),
    "w4a16_gemv_qkv_rope_f16": (
        ctypes.c_int,
        [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 6 + [_vp],
    ),
    "w4a16_attention_o_cached_f16": (ctypes.c_int, [_vp] * 7 + [_i64] * 6 + [_vp]),
    "w4a16_gemv_argmax_workspace_bytes": (_i64, [_i64]),
    "w4a16_gemv_argmax_f16": (
        ctypes.c_int,
        [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp],
    ),
    "w4a16_argmax_f16": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp]),
    "w4a16_argmax_embed_f16": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "w4a16_embed_rmsnorm_f16": (ctypes.c_int, [_vp, _i64, _i64, _vp, _i64, _vp, ctypes.c_float, _vp, _vp, _vp,
                                               _vp]),
    "w4a16_embedding_f16": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "w4a16_rmsnorm_f16": (ctypes.c_int, [_vp, _vp, ctypes.c_float, _vp, _i64, _i64, _vp]),
    "w4a16_silu_mul_f16": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp]),
    "w4a16_add_rmsnorm_f16": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_float, _vp, _vp, _i64, _i64, _vp]),
    "w4a16_linear_add_rmsnorm_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _i64, _i64,
                                                    _i64, _i64, _vp, _i64, _vp]),
    "w4a16_linear_add_rmsnorm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "w4a16_prefill_attention_o_add_rmsnorm_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                                                  _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp,
                                                                  ctypes.c_float, _vp, _vp, _vp, _i64, _vp]),
    "w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "w4a16_linear_silu_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "w4a16_prefill_attention_f16": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                                   _i64, _vp]),
}

_lib = None


class W4A16Error(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def lib() -> ctypes.CDLL:
    """Load ``libw4a16_hip.so`` (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in {**SIGNATURES, **DECODE_SIGNATURES}.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().w4a16_last_error().decode()


def _raise_on(code: int) -> None:
    if code != W4A16_OK:
        raise W4A16Error(code, last_error())


def _stream_ptr(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


def linear_workspace_bytes(m: int, n: int, k: int, group_size: int = 128) -> int:
    """Workspace bytes ``w4a16_linear_ws_f16`` uses for these sizes (host-only)."""
    return int(lib().w4a16_linear_workspace_bytes(m, n, k, group_size))


def _workspace(nbytes: int, device, stream=None):
    """An fp32 workspace from the caching allocator. When the launches run on
    a stream other than the current one, the block is recorded on that
    stream, so the allocator does not hand it out again while those launches
    may still read or write it."""
    ws = torch.empty(((nbytes + 3) // 4,), dtype=torch.float32, device=device)
    if stream is not None and stream != torch.cuda.current_stream(device):
        ws.record_stream(stream)
    return ws


def linear_f16(activations, packed_weights, scales, output, group_size: int = 128, stream=None,
               workspace="auto") -> None:
    """Run the W4A16 linear layer on torch device tensors (no checks beyond the
    C ABI's): ``w4a16_linear_ws_f16`` with a workspace from the caching
    allocator when the plan uses one (``workspace="auto"``, as the torch op
    does), a given fp32 tensor, or ``None`` for ``w4a16_linear_f16``."""
    m, k = activations.shape
    n = packed_weights.shape[0]
    if isinstance(workspace, str):
        nbytes = linear_workspace_bytes(m, n, k, group_size)
        workspace = _workspace(nbytes, output.device, stream) if nbytes > 0 else None
    if workspace is None:
        _raise_on(
            lib().w4a16_linear_f16(
                activations.data_ptr(), packed_weights.data_ptr(), scales.data_ptr(), output.data_ptr(),
                m, n, k, group_size, _stream_ptr(stream),
            )
        )
        return
    _raise_on(
        lib().w4a16_linear_ws_f16(
            activations.data_ptr(), packed_weights.data_ptr(), scales.data_ptr(), output.data_ptr(),
            m, n, k, group_size, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
            _stream_ptr(stream),
        )
    )


NOALLOC_SCRATCH_BYTES = 8 << 20   # W4A16_NOALLOC_SCRATCH_BYTES


def linear_noalloc_f16(activations, packed_weights, scales, output, group_size: int = 128, stream=None) -> None:
    """``w4a16_linear_noalloc_f16``: the default routing with the split-K
    partial sums in the library's own device scratch (no allocation)."""
    m, k = activations.shape
    n = packed_weights.shape[0]
    _raise_on(
        lib().w4a16_linear_noalloc_f16(
            activations.data_ptr(), packed_weights.data_ptr(), scales.data_ptr(), output.data_ptr(),
            m, n, k, group_size, _stream_ptr(stream),
        )
    )


def linear_f16_tuned(activations, packed_weights, scales, output, group_size, kernel, rows, splits, unroll,
                     max_blocks=0, stream=None, workspace=None) -> None:
    """``w4a16_linear_f16_tuned``; the split-K paired kernel gets a workspace
    of splits * M * N fp32 (the ring kernel over max_blocks > 1 K slices one
    of max_blocks * M * N) from the caching allocator unless one is given."""
    m, k = activations.shape
    n = packed_weights.shape[0]
    if workspace is None and kernel == KERNEL_PAIR_SPLIT:
        workspace = _workspace(max(1, splits) * m * n * 4, output.device, stream)
    if workspace is None and kernel == KERNEL_PAIR_RING and max_blocks > 1:
        workspace = _workspace(max_blocks * m * n * 4, output.device, stream)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _raise_on(
        lib().w4a16_linear_f16_tuned(
            activations.data_ptr(), packed_weights.data_ptr(), scales.data_ptr(), output.data_ptr(),
            m, n, k, group_size, _stream_ptr(stream), kernel, rows, splits, unroll, max_blocks, ws_ptr, ws_bytes,
        )
    )


def dequantize_f16(packed_weights, scales, output, group_size: int = 128, stream=None) -> None:
    n, kh = packed_weights.shape
    _raise_on(
        lib().w4a16_dequantize_f16(
            packed_weights.data_ptr(), scales.data_ptr(), output.data_ptr(), n, 2 * kh, group_size,
            _stream_ptr(stream),
        )
    )


def plan_linear(act_ptr: int, packed_ptr: int, m: int, n: int, k: int, group_size: int = 128,
                workspace: bool = False) -> dict:
    """The dispatcher's choice for these sizes/alignments (host-only, no GPU
    needed); with workspace, the choice of w4a16_linear_ws_f16 with one."""
    out = [ctypes.c_int(0) for _ in range(5)]
    fn = lib().w4a16_plan_linear_ws if workspace else lib().w4a16_plan_linear
    _raise_on(fn(act_ptr, packed_ptr, m, n, k, group_size, *[ctypes.byref(v) for v in out]))
    kernel, rows, splits, unroll, max_blocks = (v.value for v in out)
    return {"kernel": KERNEL_NAMES[kernel], "rows": rows, "splits": splits, "unroll": unroll,
            "max_blocks": max_blocks}


def check_linear_shapes(act_rows, act_cols, packed_rows, packed_cols, scale_rows, scale_cols, group_size):
    code = lib().w4a16_check_linear_shapes(
        act_rows, act_cols, packed_rows, packed_cols, scale_rows, scale_cols, group_size
    )
    return code, (last_error() if code else "")


def check_dequantize_shapes(packed_rows, packed_cols, scale_rows, scale_cols, group_size, address=0):
    code = lib().w4a16_check_dequantize_shapes(packed_rows, packed_cols, scale_rows, scale_cols, group_size,
                                               address)
    return code, (last_error() if code else "")


# ---------------------------------------------------------------- decode step --
def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def gemv_fused_f16(activations, packed_weights, scales, output, norm_weight=None, eps: float = 1e-5,
                   residual=None, paired: bool = False, group_size: int = 128, stream=None) -> None:
    """``w4a16_gemv_fused_f16``: one activation row (1-D or [1, K] fp16) through
    an INT4 layer with optional RMSNorm prologue, residual add, or paired
    [gate; up] SiLU-multiply epilogue."""
    k = activations.shape[-1]
    n = packed_weights.shape[0]
    _raise_on(
        lib().w4a16_gemv_fused_f16(
            activations.data_ptr(), _ptr(norm_weight), float(eps), packed_weights.data_ptr(), scales.data_ptr(),
            _ptr(residual), output.data_ptr(), n, k, group_size, int(bool(paired)), _stream_ptr(stream),
        )
    )


def decode_attention_f16(qkv, k_cache, v_cache, cos_table, sin_table, position, output, num_heads: int,
                         num_kv_heads: int, head_dim: int = 64, stream=None) -> None:
    """``w4a16_decode_attention_f16`` on one layer's caches [kv_heads, S, head_dim]."""
    _raise_on(
        lib().w4a16_decode_attention_f16(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
            position.data_ptr(), output.data_ptr(), num_heads, num_kv_heads, head_dim, k_cache.shape[-2],
            _stream_ptr(stream),
        )
    )


def decode_attention_split_f16(qkv, k_cache, v_cache, cos_table, sin_table, position, output, num_heads: int,
                               num_kv_heads: int, splits: int, workspace, head_dim: int = 64, stream=None) -> None:
    """``w4a16_decode_attention_split_f16``: the slots split into `splits` shares
    (one workgroup per head and share), merged per head; `workspace` holds at
    least num_heads * splits * 66 fp32."""
    _raise_on(
        lib().w4a16_decode_attention_split_f16(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
            position.data_ptr(), output.data_ptr(), num_heads, num_kv_heads, head_dim, k_cache.shape[-2], splits,
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream_ptr(stream),
        )
    )


def attention_o_f16(qkv, k_cache, v_cache, inv_freq, position, o_packed, o_scales, residual, num_heads: int,
                    num_kv_heads: int, head_dim: int = 64, group_size: int = 128, stream=None) -> None:
    """``w4a16_attention_o_f16``: one layer's attention of the new token (caches
    [kv_heads, S, head_dim], position < 64) fused with the o projection;
    residual [hidden] += o(attn) in fp16."""
    _raise_on(
        lib().w4a16_attention_o_f16(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), inv_freq.data_ptr(), position.data_ptr(),
            o_packed.data_ptr(), o_scales.data_ptr(), residual.data_ptr(), num_heads, num_kv_heads, head_dim,
            k_cache.shape[-2], residual.numel(), group_size, _stream_ptr(stream),
        )
    )


def gemv_qkv_rope_f16(activations, packed_weights, scales, qkv, k_cache, v_cache, inv_freq, position,
                      num_heads: int, num_kv_heads: int, norm_weight=None, eps: float = 1e-5, head_dim: int = 64,
                      group_size: int = 128, stream=None) -> None:
    """``w4a16_gemv_qkv_rope_f16``: RMSNorm (optional) + the q|k|v GEMV of one
    row, q / k rotated at the device position, k / v appended to the caches
    [kv_heads, S, head_dim]; qkv receives the rotated q, k and the v rows."""
    _raise_on(
        lib().w4a16_gemv_qkv_rope_f16(
            activations.data_ptr(), _ptr(norm_weight), float(eps), packed_weights.data_ptr(), scales.data_ptr(),
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), inv_freq.data_ptr(), position.data_ptr(),
            num_heads, num_kv_heads, head_dim, k_cache.shape[-2], activations.shape[-1], group_size,
            _stream_ptr(stream),
        )
    )


def attention_o_cached_f16(qkv, k_cache, v_cache, position, o_packed, o_scales, residual, num_heads: int,
                           num_kv_heads: int, head_dim: int = 64, group_size: int = 128, stream=None) -> None:
    """``w4a16_attention_o_cached_f16``: attention + o projection + residual
    after ``gemv_qkv_rope_f16`` (rotated q in qkv, slot `position` already in
    the caches; position < 64)."""
    _raise_on(
        lib().w4a16_attention_o_cached_f16(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), position.data_ptr(), o_packed.data_ptr(),
            o_scales.data_ptr(), residual.data_ptr(), num_heads, num_kv_heads, head_dim, k_cache.shape[-2],
            residual.numel(), group_size, _stream_ptr(stream),
        )
    )


def gemv_argmax_workspace_bytes(n: int) -> int:
    """Bytes of the workspace ``gemv_argmax_f16`` needs for an N-row layer."""
    return int(lib().w4a16_gemv_argmax_workspace_bytes(n))


def gemv_argmax_f16(x, packed, scales, token, workspace, logits=None, norm_weight=None, eps: float = 1e-6,
                    position=None, table=None, emb_out=None, group_size: int = 128, stream=None) -> None:
    """``w4a16_gemv_argmax_f16``: logits = W x' (RMSNorm first when norm_weight is
    given), token <- argmax, position += 1, emb_out <- table[token]; one launch.
    ``workspace``: a zeroed device tensor of at least
    ``gemv_argmax_workspace_bytes(N)`` bytes, reused across calls."""
    n, k = packed.shape[0], packed.shape[1] * 2
    vocab, hidden = (table.shape if table is not None else (0, 0))
    _raise_on(
        lib().w4a16_gemv_argmax_f16(
            x.data_ptr(), _ptr(norm_weight), eps, packed.data_ptr(), scales.data_ptr(), _ptr(logits), n, k,
            group_size, token.data_ptr(), _ptr(position), _ptr(table), vocab, hidden, _ptr(emb_out),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream_ptr(stream),
        )
    )


def argmax_f16(logits, token, position=None, stream=None) -> None:
    """``w4a16_argmax_f16``: token <- argmax(logits); position += 1 when given."""
    _raise_on(lib().w4a16_argmax_f16(logits.data_ptr(), logits.numel(), token.data_ptr(), _ptr(position),
                                     _stream_ptr(stream)))


def argmax_embed_f16(logits, token, position, table, output, stream=None, token_copy=None) -> None:
    """``w4a16_argmax_embed_f16``: token <- argmax(logits); position += 1;
    output <- table[token] (the next step's input row); token_copy (an int64
    element, e.g. a slot of a token history) <- the token as well."""
    vocab, hidden = table.shape
    _raise_on(lib().w4a16_argmax_embed_f16(logits.data_ptr(), logits.numel(), token.data_ptr(), _ptr(position),
                                           table.data_ptr(), vocab, hidden, output.data_ptr(), _ptr(token_copy),
                                           _stream_ptr(stream)))


def embed_rmsnorm_f16(table, tokens, weight, eps: float, x_out, output, position=None, stream=None) -> None:
    """``w4a16_embed_rmsnorm_f16``: x_out <- table[tokens] ([rows, hidden]);
    output <- RMSNorm(x_out) * weight; position (int64[1]) <- rows when given."""
    vocab, hidden = table.shape
    _raise_on(lib().w4a16_embed_rmsnorm_f16(table.data_ptr(), vocab, hidden, tokens.data_ptr(), tokens.numel(),
                                            weight.data_ptr(), float(eps), x_out.data_ptr(), output.data_ptr(),
                                            _ptr(position), _stream_ptr(stream)))


def embedding_f16(table, token, output, stream=None) -> None:
    """``w4a16_embedding_f16``: output <- table[token]."""
    vocab, hidden = table.shape
    _raise_on(lib().w4a16_embedding_f16(table.data_ptr(), vocab, hidden, token.data_ptr(), output.data_ptr(),
                                        _stream_ptr(stream)))


def rmsnorm_f16(x, weight, eps: float, output, stream=None) -> None:
    """``w4a16_rmsnorm_f16`` over the rows of x [rows, hidden]."""
    rows, hidden = x.shape
    _raise_on(lib().w4a16_rmsnorm_f16(x.data_ptr(), weight.data_ptr(), float(eps), output.data_ptr(), rows, hidden,
                                      _stream_ptr(stream)))


def add_rmsnorm_f16(x, delta, weight, eps: float, x_out, output, stream=None) -> None:
    """``w4a16_add_rmsnorm_f16``: x_out <- x + delta, output <- RMSNorm(x_out) * weight
    over the rows of x [rows, hidden] (x_out may be x)."""
    rows, hidden = x.shape
    _raise_on(lib().w4a16_add_rmsnorm_f16(x.data_ptr(), delta.data_ptr(), weight.data_ptr(), float(eps),
                                          x_out.data_ptr(), output.data_ptr(), rows, hidden, _stream_ptr(stream)))


def linear_silu_f16(activations, packed_weights, scales, output, group_size: int = 128, stream=None) -> None:
    """``w4a16_linear_silu_f16``: output [M, inter] <- silu(x W_gate^T) * (x W_up^T) for
    packed_weights [2 inter, K / 2] ([gate; up] rows)."""
    m, k = activations.shape
    inter = packed_weights.shape[0] // 2
    _raise_on(lib().w4a16_linear_silu_f16(activations.data_ptr(), packed_weights.data_ptr(), scales.data_ptr(),
                                          output.data_ptr(), m, inter, k, group_size, _stream_ptr(stream)))


def linear_add_rmsnorm_f16(activations, packed_weights, scales, x, norm_weight, eps: float, x_out, output,
                           group_size: int = 128, stream=None, workspace=None) -> None:
    """``w4a16_linear_add_rmsnorm_f16``: x_out <- x + linear(activations),
    output <- RMSNorm(x_out) * norm_weight, with a workspace from the caching
    allocator unless one is given."""
    m, k = activations.shape
    n = packed_weights.shape[0]
    if workspace is None:
        nbytes = int(lib().w4a16_linear_add_rmsnorm_workspace_bytes(m, n, k, group_size))
        workspace = _workspace(max(nbytes, 16), output.device, stream)
    _raise_on(lib().w4a16_linear_add_rmsnorm_f16(
        activations.data_ptr(), packed_weights.data_ptr(), scales.data_ptr(), x.data_ptr(), norm_weight.data_ptr(),
        float(eps), x_out.data_ptr(), output.data_ptr(), m, n, k, group_size, workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream_ptr(stream)))


def prefill_attention_o_add_rmsnorm_f16(qkv, k_cache, v_cache, cos_table, sin_table, start: int, o_packed,
                                        o_scales, x, norm_weight, eps: float, x_out, output, num_heads: int,
                                        num_kv_heads: int, head_dim: int = 64, group_size: int = 128, stream=None,
                                        workspace=None) -> None:
    """``w4a16_prefill_attention_o_add_rmsnorm_f16``: the attention of the
    qkv rows [tokens, ...] at slots start .. start + tokens - 1 of one
    layer's caches (appending their k / v rows), x_out <- x + linear(attn, o),
    output <- RMSNorm(x_out) * norm_weight; a workspace from the caching
    allocator unless one is given."""
    tokens = qkv.shape[0]
    hidden = o_packed.shape[0]
    if workspace is None:
        nbytes = int(lib().w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes(tokens, num_heads, hidden,
                                                                                 group_size))
        workspace = _workspace(max(nbytes, 16), output.device, stream)
    _raise_on(lib().w4a16_prefill_attention_o_add_rmsnorm_f16(
        qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(), start,
        tokens, num_heads, num_kv_heads, head_dim, k_cache.shape[-2], o_packed.data_ptr(), o_scales.data_ptr(),
        hidden, group_size, x.data_ptr(), norm_weight.data_ptr(), float(eps), x_out.data_ptr(), output.data_ptr(),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), _stream_ptr(stream)))


def silu_mul_f16(gate_up, output, stream=None) -> None:
    """``w4a16_silu_mul_f16``: output [rows, inter] <- silu(gate) * up of gate_up [rows, 2 * inter]."""
    rows, width = gate_up.shape
    _raise_on(lib().w4a16_silu_mul_f16(gate_up.data_ptr(), output.data_ptr(), rows, width // 2, _stream_ptr(stream)))


def prefill_attention_f16(qkv, k_cache, v_cache, cos_table, sin_table, start: int, output, num_heads: int,
                          num_kv_heads: int, head_dim: int = 64, stream=None) -> None:
    """``w4a16_prefill_attention_f16`` for the qkv rows [tokens, ...] at slots
    start .. start + tokens - 1 of one layer's caches [kv_heads, S, head_dim]."""
    _raise_on(
        lib().w4a16_prefill_attention_f16(
            qkv.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
            start, qkv.shape[0], output.data_ptr(), num_heads, num_kv_heads, head_dim, k_cache.shape[-2],
            _stream_ptr(stream),
        )
    )
