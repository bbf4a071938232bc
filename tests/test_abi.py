"""Host-only checks of the C ABI (no GPU): the library loads, exports every
symbol include/w4a16_hip.h declares, validates shapes with the reference's
messages, and routes calls as the reference's dispatcher does
(reference csrc/int4_linear_kernel.cu:641-802)."""

from __future__ import annotations

import os
import re

import pytest
import torch

from nibble_amd import _lib

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include")
HEADER = os.path.join(INCLUDE, "w4a16_hip.h")
DECODE_HEADER = os.path.join(INCLUDE, "w4a16_decode.h")


def declared_functions(header: str = HEADER) -> list[str]:
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(w4a16_\w+)\s*\(", text, re.M)))


@pytest.mark.parametrize("header,table,minimum", [(HEADER, "SIGNATURES", 8), (DECODE_HEADER, "DECODE_SIGNATURES", 4)])
def test_header_symbols_exported(header, table, minimum):
    names = declared_functions(header)
    assert len(names) >= minimum, names
    lib = _lib.lib()
    for name in names:
        assert hasattr(lib, name), f"{name} not exported by libw4a16_hip.so"
    assert set(names) == set(getattr(_lib, table)), "ctypes binding out of sync with the header"


def test_decode_entry_points_validate_before_launch():
    """Argument checks of include/w4a16_decode.h return codes without touching a GPU."""
    lib = _lib.lib()
    a = 1 << 20   # an aligned stand-in address; nothing is launched on these paths
    # fused GEMV: group size, K range, odd paired rows, residual with paired, alignment
    assert lib.w4a16_gemv_fused_f16(a, 0, 1e-5, a, a, 0, a, 8, 256, 64, 0, 0) == _lib.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_gemv_fused_f16(a, 0, 1e-5, a, a, 0, a, 8, 32768, 128, 0, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_gemv_fused_f16(a, 0, 1e-5, a, a, 0, a, 7, 256, 128, 1, 0) == _lib.W4A16_ERR_SHAPE
    assert "even" in _lib.last_error()
    assert lib.w4a16_gemv_fused_f16(a, 0, 1e-5, a, a, a, a, 8, 256, 128, 1, 0) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_gemv_fused_f16(a + 2, 0, 1e-5, a, a, 0, a, 8, 256, 128, 0, 0) == _lib.W4A16_ERR_ALIGNMENT
    assert lib.w4a16_gemv_fused_f16(a, 0, -1.0, a, a, 0, a, 8, 256, 128, 0, 0) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_gemv_fused_f16(0, 0, 1e-5, a, a, 0, a, 8, 256, 128, 0, 0) == _lib.W4A16_ERR_NULL
    # attention: head_dim, head grouping, sequence length, NULL pointers
    args = [a] * 7
    assert lib.w4a16_decode_attention_f16(*args, 32, 4, 128, 64, 0) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_decode_attention_f16(*args, 30, 4, 64, 64, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_decode_attention_f16(*args, 32, 4, 64, 0, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_decode_attention_f16(0, *args[1:], 32, 4, 64, 64, 0) == _lib.W4A16_ERR_NULL
    # argmax / embedding
    assert lib.w4a16_argmax_f16(a, 0, a, 0, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_argmax_f16(0, 10, a, 0, 0) == _lib.W4A16_ERR_NULL
    assert lib.w4a16_embedding_f16(a, 0, 64, a, a, 0) == _lib.W4A16_ERR_SHAPE
    # embedding rows + RMSNorm: rejects before any launch
    assert lib.w4a16_embed_rmsnorm_f16(0, 10, 64, a, 2, a, 1e-5, a, a, 0, 0) == _lib.W4A16_ERR_NULL
    assert lib.w4a16_embed_rmsnorm_f16(a, 10, 60, a, 2, a, 1e-5, a, a, 0, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_embed_rmsnorm_f16(a, 10, 16384, a, 2, a, 1e-5, a, a, 0, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_embed_rmsnorm_f16(a, 10, 64, a, 2, a, -1.0, a, a, 0, 0) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_embed_rmsnorm_f16(a + 2, 10, 64, a, 2, a, 1e-5, a, a, 0, 0) == _lib.W4A16_ERR_ALIGNMENT
    assert lib.w4a16_embed_rmsnorm_f16(a, 10, 64, a, 0, a, 1e-5, a, a, 0, 0) == _lib.W4A16_OK
    assert lib.w4a16_embedding_f16(a, 10, 64, 0, a, 0) == _lib.W4A16_ERR_NULL
    # residual add + RMSNorm: row length, NULL pointers, eps
    assert lib.w4a16_add_rmsnorm_f16(a, a, a, 1e-5, a, a, 4, 8193, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_add_rmsnorm_f16(a, 0, a, 1e-5, a, a, 4, 2048, 0) == _lib.W4A16_ERR_NULL
    assert lib.w4a16_add_rmsnorm_f16(a, a, a, -1.0, a, a, 4, 2048, 0) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_add_rmsnorm_f16(a, a, a, 1e-5, a, a, 0, 2048, 0) == _lib.W4A16_OK   # no rows: nothing
    # linear + residual add + RMSNorm: the workspace and the norm's pointers are required
    assert lib.w4a16_linear_add_rmsnorm_f16(a, a, a, a, a, 1e-5, a, a, 16, 2048, 5632, 128, 0, 0, 0) == \
        _lib.W4A16_ERR_NULL
    assert lib.w4a16_linear_add_rmsnorm_f16(a, a, a, 0, a, 1e-5, a, a, 16, 2048, 5632, 128, a, 1 << 30, 0) == \
        _lib.W4A16_ERR_NULL
    assert lib.w4a16_linear_add_rmsnorm_f16(a, a, a, a, a, 1e-5, a, a, 16, 2048, 5632, 128, a + 8, 1 << 30, 0) == \
        _lib.W4A16_ERR_ALIGNMENT
    need = lib.w4a16_linear_add_rmsnorm_workspace_bytes(16, 2048, 5632, 128)
    assert need == 8 * 16 * 2048 * 4 + 16 * 2048 * 2   # 8 K slices of partial sums, then the fp16 output
    assert lib.w4a16_linear_add_rmsnorm_workspace_bytes(4, 2048, 2048, 128) == 4 * 2048 * 2   # no K slices
    assert lib.w4a16_linear_add_rmsnorm_f16(a, a, a, a, a, 1e-5, a, a, 16, 2048, 5632, 128, a, need - 1, 0) == \
        _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_linear_add_rmsnorm_f16(a, a, a, a, a, 1e-5, a, a, 0, 2048, 5632, 128, 0, 0, 0) == _lib.W4A16_OK
    # prefill attention + o + residual add + RMSNorm: the workspace (the fused route's K slices of partial
    # sums, or the attention rows then the separate launches' workspace), pointers, alignment, empty
    need = lib.w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes(16, 32, 2048, 128)
    assert need == 8 * 16 * 2048 * 4
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes(300, 32, 2048, 128) == \
        300 * 2048 * 2 + lib.w4a16_linear_add_rmsnorm_workspace_bytes(300, 2048, 2048, 128)
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes(16, 0, 2048, 128) == 0
    attn_args = [a] * 5 + [0, 16, 32, 4, 64, 48, a, a, 2048, 128, a, a, 1e-5, a, a]
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_f16(*attn_args, 0, 0, 0) == _lib.W4A16_ERR_NULL
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_f16(*attn_args[:11], 0, *attn_args[12:], a, need, 0) == \
        _lib.W4A16_ERR_NULL
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_f16(*attn_args, a + 8, need, 0) == _lib.W4A16_ERR_ALIGNMENT
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_f16(*attn_args, a, need - 1, 0) == _lib.W4A16_ERR_CONFIG
    assert "w4a16_prefill_attention_o_add_rmsnorm_workspace_bytes" in _lib.last_error()
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_f16(*attn_args[:6], -1, *attn_args[7:], a, need, 0) == \
        _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_prefill_attention_o_add_rmsnorm_f16(*attn_args[:6], 0, *attn_args[7:], 0, 0, 0) == \
        _lib.W4A16_OK   # no tokens: nothing
    # linear + SiLU: group size, shapes, NULL pointers, alignment, empty
    assert lib.w4a16_linear_silu_f16(a, a, a, a, 4, 64, 256, 64, 0) == _lib.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_silu_f16(a, a, a, a, 4, 64, 200, 128, 0) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_linear_silu_f16(a, 0, a, a, 4, 64, 256, 128, 0) == _lib.W4A16_ERR_NULL
    assert lib.w4a16_linear_silu_f16(a + 2, a, a, a, 4, 64, 256, 128, 0) == _lib.W4A16_ERR_ALIGNMENT
    assert lib.w4a16_linear_silu_f16(a, a, a, a, 0, 64, 256, 128, 0) == _lib.W4A16_OK   # M = 0: nothing


def test_version():
    assert b"gfx950" in _lib.lib().w4a16_version()


@pytest.mark.parametrize(
    "shape,code,message",
    [
        ((1, 256, 8, 128, 8, 2, 128), _lib.W4A16_OK, ""),
        ((1, 256, 8, 128, 8, 2, 0), _lib.W4A16_ERR_GROUP_SIZE, "group_size must be greater than zero"),
        ((1, 256, 8, 128, 8, 2, 7), _lib.W4A16_ERR_GROUP_SIZE, "group_size must be even"),
        ((1, 256, 8, 64, 8, 2, 128), _lib.W4A16_ERR_SHAPE, "same K dimension"),
        ((1, 200, 8, 100, 8, 2, 128), _lib.W4A16_ERR_SHAPE, "K must be divisible by group_size"),
        ((1, 256, 8, 128, 8, 3, 128), _lib.W4A16_ERR_SHAPE, "scales must have shape [N, K / group_size]"),
        ((1, 256, 8, 128, 7, 2, 128), _lib.W4A16_ERR_SHAPE, "scales must have shape [N, K / group_size]"),
    ],
)
def test_check_linear_shapes(shape, code, message):
    got, msg = _lib.check_linear_shapes(*shape)
    assert got == code
    assert message in msg


def test_check_dequantize_shapes():
    assert _lib.check_dequantize_shapes(8, 128, 8, 2, 128, 0)[0] == _lib.W4A16_OK
    code, msg = _lib.check_dequantize_shapes(8, 48, 8, 2, 48, 0)
    assert code == _lib.W4A16_ERR_GROUP_SIZE and "multiple of 32" in msg
    code, msg = _lib.check_dequantize_shapes(8, 128, 8, 2, 128, 8)
    assert code == _lib.W4A16_ERR_ALIGNMENT and "16-byte aligned" in msg
    code, msg = _lib.check_dequantize_shapes(8, 128, 8, 4, 128, 0)
    assert code == _lib.W4A16_ERR_SHAPE


ALIGNED = 1 << 20


@pytest.mark.parametrize(
    "m,k,g,act,kernel",
    [
        (1, 2048, 128, ALIGNED, "oneshot"),    # decode
        (1, 11008, 128, ALIGNED, "oneshot"),
        (1, 32768, 128, ALIGNED, "oneshot"),   # 16 loads of 1 KiB per row (N = 64: too few rows to stream)
        (1, 34816, 128, ALIGNED, "valu"),      # rows too long for the one-shot kernel
        (2, 2048, 128, ALIGNED, "oneshot"),    # M = 2 up to K = 5632
        (2, 5632, 128, ALIGNED, "oneshot"),
        (3, 2048, 128, ALIGNED, "mfma_pair"),  # M >= 3: paired-group MFMA wherever M*K fits in LDS
        (4, 2048, 128, ALIGNED, "mfma_pair"),
        (4, 5632, 128, ALIGNED, "mfma_pair"),
        (2, 8192, 128, ALIGNED, "mfma_pair"),  # M = 2, rows above 6144 weights: the paired kernel
        (2, 28672, 128, ALIGNED, "mfma_pair"),
        (4, 8192, 128, ALIGNED, "mfma_pair"),
        (8, 8192, 128, ALIGNED, "mfma_pair"),
        (8, 8320, 128, ALIGNED, "mfma_pair"),      # rows past LDS: staged in chunks
        (4, 14336, 128, ALIGNED, "mfma_pair"),
        (4, 16384, 128, ALIGNED, "mfma_pair"),
        (8, 28672, 128, ALIGNED, "mfma_pair"),
        (8, 32768, 128, ALIGNED, "mfma_pair"),
        (8, 32896, 128, ALIGNED, "mfma"),          # beyond 16 pairs per wavefront
        (5, 2048, 128, ALIGNED, "mfma_pair"),
        (8, 4096, 128, ALIGNED, "mfma_pair"),
        (8, 5632, 128, ALIGNED, "mfma_pair"),
        (9, 2048, 128, ALIGNED, "gemm"),           # a short prompt: the GEMM at one activation tile
        (16, 4096, 128, ALIGNED, "gemm"),
        (12, 5632, 128, ALIGNED, "mfma_pair"),     # M = 9..16 on long rows: one paired launch (16 row slots)
        (9, 5632, 128, ALIGNED, "mfma_pair"),
        (9, 28672, 128, ALIGNED, "gemm"),
        (16, 34816, 128, ALIGNED, "gemm"),
        (17, 2048, 128, ALIGNED, "gemm"),          # prompts above one tile: the W4A16 GEMM
        (64, 5632, 128, ALIGNED, "gemm"),
        (300, 34816, 128, ALIGNED, "gemm"),
        (17, 2048, 128, ALIGNED + 2, "generic"),   # misaligned prompt
        (1, 2048, 64, ALIGNED, "generic"),     # group size other than 128
        (1, 2048, 128, ALIGNED + 2, "generic"),  # activations not 16-byte aligned
        (0, 2048, 128, ALIGNED, "none"),       # empty
    ],
)
def test_plan_routing(monkeypatch, m, k, g, act, kernel):
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    assert _lib.plan_linear(act, ALIGNED, m, 64, k, g)["kernel"] == kernel


@pytest.mark.parametrize("n,k,kernel,rows,splits,unroll", [
    (8192, 28672, "pair_ring", 4, 2, 6), (4096, 14336, "pair_ring", 2, 2, 10), (8192, 16384, "stream", 2, 8, 3),
    (4096, 32768, "stream", 4, 4, 2), (4096, 16512, "stream", 4, 4, 2),
    (4096, 11008, "oneshot", 1, 8, 6), (2048, 16384, "oneshot", 1, 8, 8), (28672, 8192, "pair_ring", 7, 1, 6),
    (4096, 34816, "valu", 2, 4, 8),
])
def test_stream_plan_shapes(monkeypatch, n, k, kernel, rows, splits, unroll):
    """M = 1: the paired M = 1 kernel where a launch shape is instantiated
    for the row length; other long rows of wide layers stream; shorter rows,
    narrow layers and rows past 32768 keep their kernels."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, n, k, 128)
    assert (plan["kernel"], plan["rows"], plan["splits"], plan["unroll"]) == (kernel, rows, splits, unroll)
    if kernel == "stream":
        assert plan["max_blocks"] == 0
        monkeypatch.setenv("W4A16_ROWS_PER_WARP", "2")   # an explicit VALU row count keeps auto off it
        assert _lib.plan_linear(ALIGNED, ALIGNED, 1, n, k, 128)["kernel"] != "stream"


@pytest.mark.parametrize("m,n,k,rows,blocks,splits", [
    # best shapes of the M = 32..256 sweep on the 1.1B / 8B layers
    (32, 2560, 2048, 1, 2, 4), (32, 2048, 2048, 1, 1, 4), (32, 11264, 2048, 2, 4, 4), (32, 14336, 4096, 2, 4, 4),
    (64, 2560, 2048, 2, 2, 4), (64, 2048, 5632, 1, 2, 4), (48, 11264, 2048, 2, 4, 4), (64, 4096, 14336, 2, 2, 4),
    (100, 2048, 5632, 2, 2, 4), (256, 2048, 5632, 2, 4, 4),   # from M = 64 short rows mostly take the 32x32 GEMM
    (128, 4096, 14336, 2, 4, 4),   # long rows up to M = 128: gemm_w4a16, not the staged kernel
    (17, 64, 256, 1, 1, 2),     # few workgroups whatever the shape: the most; short rows: 2 wavefronts
])
def test_gemm_plan_shapes(monkeypatch, m, n, k, rows, blocks, splits):
    """M > 16: the largest tile (activation tiles within ceil(M / 16)) that
    leaves >= 160 workgroups; 4 wavefronts splitting K, 2 on rows of fewer
    than 8 groups."""
    monkeypatch.setenv("W4A16_DECODE", "valu")   # the selector covers M <= 8 only
    plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
    assert (plan["kernel"], plan["rows"], plan["max_blocks"], plan["splits"]) == ("gemm", rows, blocks, splits)


@pytest.mark.parametrize("m,n,k,kernel,waves", [
    (8, 28672, 8192, "pair_stream", 16), (4, 28672, 8192, "pair_stream", 16), (8, 14336, 4096, "pair_ring", 0),
    (3, 14336, 4096, "pair_ring", 0), (4, 14336, 14336, "pair_stream", 8),
    (8, 14336, 14336, "mfma_pair", 0),    # 8 x 14336 activations do not fit in LDS
    (8, 8192, 8192, "pair_ring", 0), (8, 14336, 2048, "mfma_pair", 0), (2, 28672, 8192, "pair_stream", 16),
    (2, 14336, 4096, "pair_ring", 0), (5, 14336, 8192, "pair_stream", 8),
])
def test_pair_stream_routing(monkeypatch, m, n, k, kernel, waves):
    """M >= 3 on wide layers (N >= 14336, K >= 4096) whose activations fit
    in LDS and that the ring kernel does not take: the streaming paired
    kernel, 4 pairs in flight, 16 wavefronts from 3072 row blocks of 8, else
    8."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
    assert plan["kernel"] == kernel
    if kernel == "pair_stream":
        assert (plan["rows"], plan["unroll"], plan["max_blocks"]) == (waves, 4, 0)
    monkeypatch.setenv("W4A16_DECODE", "pair_stream")   # any layer whose activations fit
    assert _lib.plan_linear(ALIGNED, ALIGNED, 4, 64, 2048, 128)["kernel"] == "pair_stream"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 8, 64, 16384, 128)["kernel"] == "mfma_pair"   # too long for LDS


@pytest.mark.parametrize("m,n,k,kernel,shape", [
    (256, 14336, 4096, "gemm32", (4, 1, 4, 1)), (256, 11264, 2048, "gemm32", (4, 1, 4, 1)),
    (256, 5632, 2048, "gemm32", (2, 1, 4, 2)), (128, 14336, 4096, "gemm32", (2, 1, 4, 2)),
    (127, 14336, 4096, "gemm32", (2, 1, 4, 2)), (64, 11264, 2048, "gemm32", (2, 1, 2, 4)),
    (256, 2560, 2048, "gemm32", (2, 1, 2, 4)), (64, 5632, 2048, "gemm32", (2, 1, 1, 4)),
    (256, 2048, 2048, "gemm32", (2, 1, 1, 4)), (1024, 2048, 2048, "gemm32", (2, 1, 4, 2)),
    (512, 14336, 4096, "gemm32", (4, 2, 4, 1)), (512, 11264, 2048, "gemm32", (4, 2, 4, 1)),
    (256, 32000, 2048, "gemm32", (4, 2, 4, 1)), (255, 32000, 2048, "gemm32", (4, 1, 4, 1)),
    (512, 4096, 14336, "gemm32", (2, 1, 4, 2)), (512, 2048, 5632, "gemm32", (2, 1, 2, 4)),
    (1024, 4096, 14336, "gemm32", (4, 1, 4, 1)), (512, 28672, 8192, "gemm32", (4, 2, 4, 1)),
    (512, 1000, 5632, "gemm", None),   # long rows: no (2, 1, 1, 4); the others stay under 160 workgroups
    (511, 4096, 14336, "gemm_lds", (4, 2, 2, 4)),
    (128, 2048, 2048, "gemm", None),   # no 32x32 shape reaches 160 workgroups
    (64, 4096, 4096, "gemm", None), (32, 11264, 2048, "gemm", None), (63, 14336, 4096, "gemm", None),
    (256, 4096, 14336, "gemm_lds", (4, 2, 2, 4)), (129, 4096, 14336, "gemm_lds", (4, 2, 2, 4)),
    (128, 4096, 14336, "gemm", None),
    (256, 2048, 5632, "gemm", None),   # long rows of a narrow layer: the per-round barriers lose
])
def test_gemm_lds_routing(monkeypatch, m, n, k, kernel, shape):
    """M >= 64 on rows of up to 4096 weights, and M >= 512 on any rows: the
    32x32 staged GEMM, the first of (rows, max_blocks, unroll = wavefronts
    sharing the staging, splits) = (4, 2, 4, 1) (M >= 256), (4, 1, 4, 1),
    (2, 1, 4, 2), (2, 1, 2, 4), (2, 1, 1, 4) (rows of up to 4096 weights)
    with >= 160 workgroups; M > 128 on longer rows of layers with N >= 4096:
    the 16x16 staged GEMM, 4 activation and 2 weight tiles per wavefront;
    else gemm_w4a16."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
    assert plan["kernel"] == kernel
    if shape:
        assert (plan["rows"], plan["max_blocks"], plan["unroll"], plan["splits"]) == shape


@pytest.mark.parametrize("k,n,shape", [
    (2048, 4096, (3, 1, 7)), (2048, 5632, (3, 1, 7)), (2048, 8191, (3, 1, 7)), (2048, 8192, (3, 1, 6)),
    (2048, 16383, (3, 1, 6)), (2048, 16384, (8, 1, 4)),
    (2048, 32000, (8, 1, 4)), (4096, 4096, (2, 2, 7)), (4096, 8191, (2, 2, 7)), (4096, 8192, (8, 1, 6)),
    (4096, 14336, (8, 1, 6)), (3840, 14336, (2, 2, 7)),   # 15 pairs: 8 per wavefront over 2 slices
    (5632, 2048, (1, 4, 6)), (6144, 4096, (1, 4, 6)), (5376, 2048, (1, 4, 6)), (8192, 8192, (4, 2, 6)),
    (8192, 4096, (4, 2, 6)), (8192, 28672, (7, 1, 6)), (7936, 8192, (4, 2, 6)), (14336, 4096, (2, 2, 10)),
    (14080, 8192, (2, 2, 10)), (28672, 8192, (4, 2, 6)), (28416, 4096, (4, 2, 6)),
])
def test_pair_ring_m1_plan_shapes(monkeypatch, k, n, shape):
    """M = 1, group 128, aligned operands: the paired M = 1 kernel with the
    launch shape (rows = 8-row-block wavefronts, splits = K slices, unroll =
    pairs in flight) of its row-length class."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, n, k, 128)
    assert (plan["kernel"], plan["rows"], plan["splits"], plan["unroll"]) == ("pair_ring", *shape), (k, n)


@pytest.mark.parametrize("m,k,n,shape", [
    (2, 2048, 2048, (1, 4, 2)), (8, 2048, 1024, (1, 4, 2)), (4, 2048, 5632, (4, 1, 7)), (8, 2048, 8192, (4, 1, 6)),
    (5, 2048, 5632, (4, 1, 6)), (2, 4096, 4096, (2, 2, 6)), (8, 4096, 4096, (2, 4, 4)), (5, 4096, 6000, (2, 4, 4)), (3, 4096, 14336, (8, 1, 6)),
    (8, 4096, 28672, (8, 1, 6)), (3, 5632, 2048, (1, 8, 3)), (4, 6144, 4096, (1, 8, 3)), (2, 8192, 8192, (4, 2, 4)),
    (8, 8192, 6144, (4, 2, 5)), (5, 8192, 8192, (4, 2, 5)), (4, 8192, 8192, (4, 2, 4)), (2, 14336, 4096, (2, 4, 6)),
    (4, 14336, 8192, (2, 4, 6)),
])
def test_pair_ring_small_batch_plan_shapes(monkeypatch, m, k, n, shape):
    """M = 2..8: the ring kernel's (rows, splits, unroll) per row-length
    class and row slots (4 up to M = 4, 8 beyond)."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
    assert (plan["kernel"], plan["rows"], plan["splits"], plan["unroll"]) == ("pair_ring", *shape), (m, k, n)


def test_pair_ring_m1_plan_exclusions(monkeypatch):
    """Shapes the ring kernel leaves alone: narrow layers of short rows,
    K not a multiple of 256 or with no instantiated pairs per wavefront,
    narrow layers at M = 2, long rows at M > 4, other group sizes,
    W4A16_ROWS_PER_WARP and v1..v3; W4A16_DECODE=pair_ring selects it where
    a shape exists."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    for m, k, n in [(1, 2048, 2048), (1, 2048, 2560), (1, 4096, 2048), (1, 5632, 1024), (1, 14336, 2048),
                    (1, 2176, 8192), (1, 11008, 4096), (1, 16384, 8192), (2, 5632, 2048), (8, 14336, 4096)]:
        assert _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)["kernel"] != "pair_ring", (m, k, n)
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 14336, 4096, 64)["kernel"] == "generic"
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "2")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 14336, 4096, 128)["kernel"] == "valu"
    monkeypatch.delenv("W4A16_ROWS_PER_WARP")
    monkeypatch.setenv("W4A16_DECODE", "v3")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 14336, 4096, 128)["kernel"] == "valu_offset"
    monkeypatch.setenv("W4A16_DECODE", "pair_ring")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 14336, 4096, 128)["kernel"] == "pair_ring"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["kernel"] == "oneshot"   # no shape for N = 64
    assert _lib.plan_linear(ALIGNED, ALIGNED, 8, 14336, 14336, 128)["kernel"] == "mfma_pair"   # no shape


def test_stream_env_selector(monkeypatch):
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    monkeypatch.setenv("W4A16_DECODE", "stream")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 4096, 128)["kernel"] == "stream"     # any N
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["kernel"] == "stream"     # rows shorter than the ring
    assert _lib.plan_linear(ALIGNED, ALIGNED, 2, 64, 4096, 128)["kernel"] == "oneshot"    # M > 1
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 34816, 128)["kernel"] == "valu"      # rows too long


def test_plan_misaligned_weights_take_generic():
    assert _lib.plan_linear(ALIGNED, ALIGNED + 8, 1, 64, 2048, 128)["kernel"] == "generic"


def test_mfma_pair_plan_shapes(monkeypatch):
    monkeypatch.setenv("W4A16_DECODE", "mfma_pair")   # wide layers default to the streaming paired kernel
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    # (M, N, K) -> (splits, row-block wavefronts per workgroup, unroll, staged pairs per chunk)
    for m, n, k, splits, blocks, unroll, chunk in [
            (8, 2048, 2048, 4, 1, 2, 8), (8, 5632, 2048, 2, 4, 4, 8), (8, 4096, 4096, 4, 2, 4, 16),
            (8, 14336, 4096, 2, 8, 8, 16),                     # whole rows up to 16 pairs
            (8, 2048, 5632, 8, 1, 3, 8), (8, 8192, 8192, 4, 4, 8, 8), (8, 28672, 8192, 4, 4, 8, 8),
            (8, 4096, 14336, 8, 2, 7, 8), (8, 8192, 28672, 8, 2, 14, 8), (5, 300, 16512, 8, 1, 10, 8),
            (4, 28672, 8192, 4, 2, 8, 32),                     # two whole-row workgroups per CU
            (4, 8192, 8192, 4, 4, 8, 8), (4, 2048, 5632, 8, 1, 3, 24), (3, 6000, 14336, 8, 2, 7, 8),
            (6, 64, 128, 4, 1, 1, 4)]:
        plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
        assert (plan["kernel"], plan["splits"], plan["max_blocks"], plan["unroll"], plan["rows"]) == \
            ("mfma_pair", splits, blocks, unroll, chunk), (m, n, k)
    monkeypatch.setenv("W4A16_DECODE", "mfma_pair")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 2, 64, 2048, 128)["kernel"] == "mfma_pair"
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 2, 64, 32768, 128)
    assert (plan["kernel"], plan["splits"], plan["unroll"], plan["rows"]) == ("mfma_pair", 8, 16, 8)
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["kernel"] == "mfma"   # M = 1
    assert _lib.plan_linear(ALIGNED, ALIGNED, 8, 64, 32896, 128)["kernel"] == "mfma"   # too long
    monkeypatch.delenv("W4A16_DECODE")
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "2")   # read at M = 1 only, as in the reference
    assert _lib.plan_linear(ALIGNED, ALIGNED, 4, 64, 2048, 128)["kernel"] == "mfma_pair"


def test_mfma_oneshot_plan_shapes(monkeypatch):
    monkeypatch.setenv("W4A16_DECODE", "mfma_oneshot")
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    for m, n, k, rows, splits, unroll in [(8, 2048, 2048, 1, 4, 4), (8, 5632, 2048, 2, 4, 4),
                                          (8, 14336, 4096, 2, 4, 8), (8, 4096, 4096, 1, 8, 4),
                                          (3, 8192, 8192, 1, 8, 8), (8, 28672, 8192, 2, 8, 8),
                                          (3, 64, 128, 1, 4, 1), (5, 100, 1152, 1, 4, 3)]:
        plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
        assert (plan["kernel"], plan["rows"], plan["splits"], plan["unroll"]) == \
            ("mfma_oneshot", rows, splits, unroll), (m, n, k)
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["kernel"] == "mfma_oneshot"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 8, 64, 8320, 128)["kernel"] == "mfma"   # rows too long


def test_m2_routing(monkeypatch):
    """M = 2: the ring kernel where it has a shape; the paired kernel on
    wide layers of rows up to 4096 weights and on rows above 6144, the
    streaming paired kernel on wide layers of rows above 4096, else the
    one-shot kernel."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    for k, n, kernel in [(2048, 2048, "pair_ring"), (2048, 5632, "pair_ring"), (5632, 2048, "oneshot"),
                         (2048, 8191, "pair_ring"), (2048, 8193, "mfma_pair"), (2048, 32000, "mfma_pair"),
                         (4096, 4096, "pair_ring"), (4096, 14336, "pair_ring"), (4096, 28672, "pair_ring"),
                         (5632, 8192, "oneshot"), (6144, 8192, "oneshot"), (6272, 4096, "mfma_pair"),
                         (5632, 14336, "pair_stream"), (8192, 8192, "pair_ring"), (2048, 512, "oneshot"),
                         (8192, 14336, "pair_stream"), (14336, 4096, "pair_ring"), (28672, 2048, "mfma_pair"),
                         (28672, 28672, "mfma_pair"),   # 2 x 28672 activations past the streaming kernel's LDS
                         (34816, 64, "mfma")]:
        assert _lib.plan_linear(ALIGNED, ALIGNED, 2, n, k, 128)["kernel"] == kernel, (k, n)
    monkeypatch.setenv("W4A16_DECODE", "oneshot")   # an explicit family keeps its kernel
    assert _lib.plan_linear(ALIGNED, ALIGNED, 2, 32000, 2048, 128)["kernel"] == "oneshot"


def test_short_prompt_routing(monkeypatch):
    """M = 9..16: the paired ring kernel's 16-row-slot form on rows of 2048
    weights of 1024 .. 16384-row layers; the 16-row-slot paired kernel on
    rows longer than 4096 weights whose plan keeps 2 wavefronts or fewer on
    weight blocks (8192 x 8192 would take 4 and spill), else the GEMM; all
    three put the dequantized fp16 weights in B. The offset-decode one-shot
    MFMA kernel only with its selector. (Without a workspace: the ring
    kernel's K-slice plans need one.)"""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    for m, k, n, kernel in [(12, 2048, 8192, "pair_ring"), (16, 2048, 32000, "gemm"), (16, 2048, 512, "gemm"),
                            (9, 1024, 16384, "gemm"), (12, 2048, 4096, "pair_ring"), (16, 2048, 2560, "pair_ring"),
                            (16, 2048, 2048, "pair_ring"), (16, 2048, 11264, "pair_ring"),
                            (16, 4096, 14336, "gemm"), (16, 8192, 8192, "gemm"), (12, 8192, 4096, "mfma_pair"),
                            (9, 14336, 4096, "mfma_pair"), (12, 5632, 2048, "mfma_pair"), (17, 2048, 8192, "gemm")]:
        assert _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)["kernel"] == kernel, (m, k, n)
    monkeypatch.setenv("W4A16_DECODE", "mfma_oneshot")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 12, 8192, 2048, 128)["kernel"] == "mfma_oneshot"


def test_oneshot_plan_shapes(monkeypatch):
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    # (K, rows, waves per workgroup, loads per row) on a narrow layer
    for k, rows, splits, loads in [(2048, 1, 8, 1), (4096, 2, 8, 2), (5632, 1, 8, 3), (8192, 1, 8, 4),
                                   (14336, 1, 8, 7), (18432, 1, 8, 10), (28672, 2, 4, 14), (32768, 2, 4, 16),
                                   (256, 1, 8, 1)]:
        plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, k, 128)
        assert (plan["kernel"], plan["rows"], plan["splits"], plan["unroll"]) == ("oneshot", rows, splits, loads), k
    # wide layers the paired M = 1 kernel does not take: more rows per
    # wavefront on short rows above N = 8192
    for k, n, rows, splits, loads in [(2048, 2560, 1, 8, 1), (2048, 4095, 1, 8, 1), (1024, 32000, 4, 4, 1),
                                      (1024, 24576, 4, 4, 1), (4096, 4095, 2, 8, 2), (11008, 8192, 1, 8, 6)]:
        plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, n, k, 128)
        assert (plan["kernel"], plan["rows"], plan["splits"], plan["unroll"]) == \
            ("oneshot", rows, splits, loads), (k, n)
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 2, 2048, 5632, 128)   # M = 2: one row per wavefront
    assert (plan["kernel"], plan["rows"], plan["splits"]) == ("oneshot", 1, 8)
    assert _lib.plan_linear(ALIGNED, ALIGNED, 3, 6000, 34816, 128)["kernel"] == "mfma"     # M > 2, long rows
    assert _lib.plan_linear(ALIGNED, ALIGNED, 2, 6000, 5632, 128)["kernel"] == "oneshot"   # M = 2, any N
    monkeypatch.setenv("W4A16_DECODE", "oneshot")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 3, 6000, 2048, 128)["kernel"] == "oneshot"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 5, 64, 2048, 128)["kernel"] == "valu"     # M > 4
    assert _lib.plan_linear(ALIGNED, ALIGNED, 4, 64, 32768, 128)["kernel"] == "mfma"    # no LDS room: MFMA
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "4")
    # 4 rows (with 4 wavefronts) on rows of up to 8 loads, else 2
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)
    assert (plan["rows"], plan["splits"]) == (4, 4)
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 18432, 128)["rows"] == 2
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "2")
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)
    assert (plan["rows"], plan["splits"]) == (2, 8)


def test_env_selectors(monkeypatch):
    monkeypatch.setenv("W4A16_DECODE", "mfma")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["kernel"] == "mfma"
    monkeypatch.setenv("W4A16_DECODE", "valu")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 4, 64, 2048, 128)["kernel"] == "valu"
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "4")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["rows"] == 4
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "3")
    with pytest.raises(_lib.W4A16Error, match="W4A16_ROWS_PER_WARP must be 1, 2, or 4"):
        _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "2")
    monkeypatch.setenv("W4A16_DECODE", "v9")   # unknown values are the default, as in the reference
    monkeypatch.delenv("W4A16_ROWS_PER_WARP")
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)["kernel"] == "oneshot"


@pytest.mark.parametrize("value,kernel", [("v1", "valu"), ("v2", "diag"), ("v3", "valu_offset")])
def test_reference_decode_versions(monkeypatch, value, kernel):
    """Reference csrc/int4_linear_kernel.cu:464-476: v1..v3 pick M = 1
    variants (one row per wavefront here) on the tuned path and nothing
    else; W4A16_ROWS_PER_WARP is not read under them (:713-749)."""
    monkeypatch.setenv("W4A16_DECODE", value)
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "3")   # ignored under v1..v3
    plan = _lib.plan_linear(ALIGNED, ALIGNED, 1, 2048, 2048, 128)
    assert (plan["kernel"], plan["rows"]) == (kernel, 1)
    monkeypatch.delenv("W4A16_ROWS_PER_WARP")
    for m, k, n in [(1, 256, 7), (1, 5632, 2048), (1, 28672, 64)]:
        assert _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)["kernel"] == kernel
    # M > 1, misaligned operands, other group sizes: the default routing
    assert _lib.plan_linear(ALIGNED, ALIGNED, 4, 64, 2048, 128)["kernel"] == "mfma_pair"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 16, 64, 2048, 128)["kernel"] == "gemm"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 16, 64, 5632, 128)["kernel"] == "mfma_pair"   # 16 row slots
    assert _lib.plan_linear(ALIGNED + 2, ALIGNED, 1, 64, 2048, 128)["kernel"] == "generic"
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 64)["kernel"] == "generic"
    # activations past LDS: the default routing
    assert _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 131072, 128)["kernel"] == "mfma"


def test_reference_v4_and_default_match(monkeypatch):
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    shapes = [(1, 2048, 2048), (1, 4096, 14336), (1, 14336, 4096), (4, 2048, 5632), (8, 28672, 8192),
              (64, 2048, 2048)]
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    default = [_lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128) for m, k, n in shapes]
    for value in ("v4", "auto", "", "V4", "nonsense"):
        monkeypatch.setenv("W4A16_DECODE", value)
        assert [_lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128) for m, k, n in shapes] == default, value


def test_rows_per_warp_read_only_where_the_reference_reads_it(monkeypatch):
    """Reference :713-749 reads W4A16_ROWS_PER_WARP only for M = 1 on the
    warp kernels with the default selector: a bad value raises there and is
    ignored everywhere else."""
    monkeypatch.delenv("W4A16_DECODE", raising=False)
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "3")
    with pytest.raises(_lib.W4A16Error, match="W4A16_ROWS_PER_WARP must be 1, 2, or 4"):
        _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)
    monkeypatch.setenv("W4A16_DECODE", "v4")
    with pytest.raises(_lib.W4A16Error, match="W4A16_ROWS_PER_WARP must be 1, 2, or 4"):
        _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)
    for m in (2, 4, 8, 9, 64):   # small batch and prompts
        _lib.plan_linear(ALIGNED, ALIGNED, m, 64, 2048, 128)
    _lib.plan_linear(ALIGNED + 2, ALIGNED, 1, 64, 2048, 128)   # misaligned: the generic kernel
    _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 64)        # group size other than 128
    _lib.plan_linear(ALIGNED, ALIGNED, 0, 64, 2048, 128)       # empty
    monkeypatch.setenv("W4A16_DECODE", "v1")
    _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "")   # atoi("") = 0, rejected as in the reference
    monkeypatch.setenv("W4A16_DECODE", "v4")
    with pytest.raises(_lib.W4A16Error):
        _lib.plan_linear(ALIGNED, ALIGNED, 1, 64, 2048, 128)


def test_valu_falls_back_to_mfma_when_activations_exceed_lds(monkeypatch):
    monkeypatch.setenv("W4A16_DECODE", "valu")
    # M=8, K=14336 -> 229 KiB of activations, more than the 160 KiB of LDS
    assert _lib.plan_linear(ALIGNED, ALIGNED, 8, 64, 14336, 128)["kernel"] == "mfma"


def test_noalloc_rejects_before_launch():
    """w4a16_linear_noalloc_f16 checks its arguments on the host (nothing
    launched, so stand-in addresses are safe). The scratch holds the split-K
    partials of M = 8, K = 20480 up to N = 65536; wider layers take the route
    without a workspace (tested on the GPU)."""
    lib = _lib.lib()
    assert lib.w4a16_linear_noalloc_f16(None, None, None, None, 1, 8, 256, 0, None) == _lib.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_noalloc_f16(None, None, None, None, 1, 8, 256, 128, None) == _lib.W4A16_ERR_NULL
    assert lib.w4a16_linear_noalloc_f16(None, None, None, None, 0, 8, 256, 128, None) == _lib.W4A16_OK
    m, k = 8, 20480
    assert _lib.linear_workspace_bytes(m, 65544, k) > _lib.NOALLOC_SCRATCH_BYTES
    assert _lib.linear_workspace_bytes(m, 65536, k) == _lib.NOALLOC_SCRATCH_BYTES   # the largest that fits


def test_scalar_argument_errors():
    lib = _lib.lib()
    assert lib.w4a16_linear_f16(None, None, None, None, 1, 8, 256, 0, None) == _lib.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_f16(None, None, None, None, 1, 8, 200, 128, None) == _lib.W4A16_ERR_SHAPE
    assert lib.w4a16_linear_f16(None, None, None, None, 1, 8, 256, 128, None) == _lib.W4A16_ERR_NULL
    # empty work: nothing to launch, NULL pointers allowed
    assert lib.w4a16_linear_f16(None, None, None, None, 0, 8, 256, 128, None) == _lib.W4A16_OK
    assert lib.w4a16_dequantize_f16(None, None, None, 8, 256, 48, None) == _lib.W4A16_ERR_GROUP_SIZE
    assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 1, 8, 256, 128, None,
                                      _lib.KERNEL_VALU, 3, 1, 1, 0, None, 0) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 1, 8, 256, 64, None,
                                      _lib.KERNEL_MFMA, 1, 1, 1, 0, None, 0) == _lib.W4A16_ERR_CONFIG
    # the split-K family without (or with too small) a workspace
    assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 8, 4096, 28672, 128, None,
                                      _lib.KERNEL_PAIR_SPLIT, 0, 8, 4, 0, None, 0) == _lib.W4A16_ERR_CONFIG
    assert "workspace" in _lib.last_error()
    assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 8, 4096, 28672, 128, None,
                                      _lib.KERNEL_PAIR_SPLIT, 0, 8, 4, 0, ALIGNED, 1024) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_linear_ws_f16(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 8, 8192, 28672, 128, ALIGNED, 1024,
                                   None) == _lib.W4A16_ERR_CONFIG
    assert "workspace" in _lib.last_error()
    # slices that leave one empty, or a slice too long for LDS
    for splits in (1, 17):
        assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 8, 4096, 28672, 128, None,
                                          _lib.KERNEL_PAIR_SPLIT, 0, splits, 4, 0, ALIGNED,
                                          1 << 30) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 8, 4096, 1024, 128, None,
                                      _lib.KERNEL_PAIR_SPLIT, 0, 5, 4, 0, ALIGNED, 1 << 30) == _lib.W4A16_ERR_CONFIG
    assert lib.w4a16_linear_f16_tuned(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 8, 4096, 28672, 128, None,
                                      _lib.KERNEL_PAIR_SPLIT, 0, 2, 4, 0, ALIGNED, 1 << 30) == _lib.W4A16_ERR_CONFIG
    assert "LDS" in _lib.last_error()


@pytest.mark.parametrize("m,n,k,splits", [
    (8, 8192, 28672, 8), (8, 4096, 14336, 8), (5, 2048, 14336, 8), (8, 8192, 14336, 0), (4, 8192, 28672, 4),
    (3, 8192, 28672, 4),
    (3, 4096, 14336, 0), (5, 8192, 20480, None), (5, 4096, 20480, 0), (8, 8191, 28672, 8), (8, 8192, 16384, 0),
    (8, 2048, 5632, 0), (8, 28672, 8192, 2), (5, 16384, 8192, 2), (4, 28672, 8192, 0), (1, 8192, 28672, 0),
    (2, 8192, 28672, 0), (16, 8192, 28672, 0), (8, 4096, 4096, 0), (4, 4096, 8192, 0), (16, 2048, 5632, 8),
    (12, 4096, 14336, 4), (16, 8192, 8192, 2), (9, 2048, 5632, 0)])
def test_linear_workspace_bytes(m, n, k, splits):
    """Layers whose route keeps fp32 partial sums use slices * M * N * 4
    bytes of workspace: the paired ring kernel's K slices (M = 3..8 on rows
    of 28672 with N = 4096..8192, M = 5..8 on rows of 8192 with N >= 16384
    and on rows of 14336 with N = 2048..4096, M = 12..16 on 5632 x 2048,
    14336 x 4096 and 8192 x 8192) and the split-K
    streaming kernel (other M = 3..8 layers with K > 16384 and N >= 8192;
    None: any slice count); everything else none."""
    got = _lib.linear_workspace_bytes(m, n, k)
    if splits == 0:
        assert got == 0
    elif splits is None:
        assert got > 0 and got % (m * n * 4) == 0
        s = got // (m * n * 4)
        assert 2 <= s <= 16
    else:
        assert got == splits * m * n * 4
    assert _lib.linear_workspace_bytes(m, n, k, 64) == 0   # other group sizes: the generic kernel


def test_torch_op_schemas_match_reference():
    import nibble_amd  # noqa: F401  (registers the ops)

    assert str(torch.ops.w4a16.linear.default._schema) == (
        "w4a16::linear(Tensor activations, Tensor packed_weights, Tensor scales, int group_size) -> Tensor")
    assert str(torch.ops.w4a16.dequantize.default._schema) == (
        "w4a16::dequantize(Tensor packed_weights, Tensor scales, int group_size) -> Tensor")


def test_torch_op_rejects_cpu_tensors():
    import nibble_amd

    assert nibble_amd.cuda_extension_available()
    x = torch.zeros((1, 256), dtype=torch.float16)
    p = torch.zeros((8, 128), dtype=torch.uint8)
    s = torch.ones((8, 2), dtype=torch.float16)
    with pytest.raises(RuntimeError):
        nibble_amd.linear_cuda(x, p, s, 128)
    with pytest.raises(RuntimeError):
        nibble_amd.dequantize_cuda(p, s, 128)


def test_fake_kernels_give_shapes():
    import nibble_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty((3, 256), dtype=torch.float16, device="cuda")
        p = torch.empty((8, 128), dtype=torch.uint8, device="cuda")
        s = torch.empty((8, 2), dtype=torch.float16, device="cuda")
        y = torch.ops.w4a16.linear(x, p, s, 128)
        w = torch.ops.w4a16.dequantize(p, s, 128)
    assert tuple(y.shape) == (3, 8) and y.dtype == torch.float16
    assert tuple(w.shape) == (8, 256) and w.dtype == torch.float16


def test_split_plans_are_launchable():
    """Every split-K plan the router can make (M = 3..8, K = 16512..65536 and
    beyond) is one the launcher accepts: 2..16 slices, none empty, a slice's
    staging within 160 KiB of LDS (8 row slots for M > 4, else 4); past
    K = 65536 no workspace is asked for."""
    for m in range(3, 9):
        slots = 8 if m > 4 else 4
        for k in list(range(16512, 65537, 1152)) + [65536, 65664, 131072]:
            ws = _lib.linear_workspace_bytes(m, 8192, k)
            if k > 65536:
                assert ws == 0, (m, k)
                continue
            assert ws > 0 and ws % (m * 8192 * 4) == 0, (m, k)
            s = ws // (m * 8192 * 4)
            pairs = (k // 128 + 1) // 2
            per_slice = -(-pairs // s)
            assert 2 <= s <= 16 and (s - 1) * per_slice < pairs, (m, k, s)
            assert per_slice * 16 * (2 * slots) * 16 + per_slice * 128 <= 160 * 1024, (m, k, s)


@pytest.mark.parametrize("m,k,n,sk,sn,depth,slices", [
    (8, 28672, 8192, 1, 8, 2, 8), (5, 28672, 8192, 1, 8, 2, 8), (3, 28672, 8192, 1, 8, 4, 4),
    (8, 8192, 28672, 1, 8, 3, 2), (16, 5632, 2048, 1, 8, 3, 8), (12, 14336, 4096, 1, 8, 4, 4),
    (16, 8192, 8192, 1, 8, 4, 2)])
def test_workspace_plan_ring_slices(m, k, n, sk, sn, depth, slices):
    """w4a16_plan_linear_ws: the route w4a16_linear_ws_f16 takes with a
    workspace, here the ring kernel over K slices (max_blocks = slices);
    without one the same layers plan no K slices."""
    plan = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128, workspace=True)
    assert plan == {"kernel": "pair_ring", "rows": sn, "splits": sk, "unroll": depth, "max_blocks": slices}
    plain = _lib.plan_linear(ALIGNED, ALIGNED, m, n, k, 128)
    assert not (plain["kernel"] == "pair_ring" and plain["max_blocks"] > 1)
