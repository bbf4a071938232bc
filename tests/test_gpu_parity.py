"""GPU parity of the HIP kernels, called through the C ABI (ctypes), against
the CPU oracle. Bar: |err| <= 1e-2 (1 + |ref|) for the linear layer, bit
identity for dequantize."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from nibble_amd import _lib
from tests._cases import assert_parity, expected, make_case

pytestmark = pytest.mark.gpu

VALU, MFMA, GENERIC, DIAG = _lib.KERNEL_VALU, _lib.KERNEL_MFMA, _lib.KERNEL_GENERIC, _lib.KERNEL_DIAG
VOFF = _lib.KERNEL_VALU_OFFSET
ONESHOT = _lib.KERNEL_ONESHOT
MFMA_OS = _lib.KERNEL_MFMA_ONESHOT
MFMA_PAIR = _lib.KERNEL_MFMA_PAIR
STREAM = _lib.KERNEL_STREAM
GEMM = _lib.KERNEL_GEMM
PAIR_STREAM = _lib.KERNEL_PAIR_STREAM
GEMM_LDS = _lib.KERNEL_GEMM_LDS
GEMM32 = _lib.KERNEL_GEMM32
PAIR_SPLIT = _lib.KERNEL_PAIR_SPLIT


def _run_tuned(dev, x, packed, scales, kernel, rows, splits, unroll, max_blocks=0, group_size=128):
    xd, pd, sd = x.to(dev), packed.to(dev), scales.to(dev)
    out = torch.full((x.shape[0], packed.shape[0]), float("nan"), dtype=torch.float16, device=dev)
    print(f"[case] kernel={kernel} rows={rows} splits={splits} unroll={unroll} max_blocks={max_blocks} "
          f"M={x.shape[0]} K={x.shape[1]} N={packed.shape[0]}", flush=True)
    _lib.linear_f16_tuned(xd, pd, sd, out, group_size, kernel, rows, splits, unroll, max_blocks)
    torch.cuda.synchronize()
    return out


def _run_default(dev, x, packed, scales, group_size=128, workspace="auto"):
    xd, pd, sd = x.to(dev), packed.to(dev), scales.to(dev)
    out = torch.full((x.shape[0], packed.shape[0]), float("nan"), dtype=torch.float16, device=dev)
    print(f"[case] default M={x.shape[0]} K={x.shape[1]} N={packed.shape[0]} G={group_size} ws={workspace is not None}",
          flush=True)
    _lib.linear_f16(xd, pd, sd, out, group_size, workspace=workspace)
    torch.cuda.synchronize()
    return out


# ---- shapes from the reference's GPU tests and the benchmark configs ----
SHAPES_M1 = [(256, 8), (256, 7), (1024, 13), (2048, 2048), (2048, 5632), (5632, 2048)]


@pytest.mark.parametrize("k,n", SHAPES_M1)
def test_default_dispatch_m1(gpu, k, n):
    x, p, s = make_case(1, k, n, seed=k + n)
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M=1 K={k} N={n}")


@pytest.mark.parametrize("m", [2, 3, 4, 5, 6, 7, 8])
def test_default_dispatch_small_batch(gpu, m):
    x, p, s = make_case(m, 2048, 2048, seed=m)
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M={m}")


@pytest.mark.parametrize("m", [2, 4, 8])
@pytest.mark.parametrize("k,n", [(2048, 2048), (2048, 5632), (5632, 2048)])
def test_default_dispatch_configs2(gpu, m, k, n):
    """every M in {2, 4, 8} on its three layer shapes, at full size,
    through the default route the benchmark times."""
    x, p, s = make_case(m, k, n, seed=100 * m + k + n)
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"configs2 M={m} K={k} N={n}")


@pytest.mark.parametrize("m", [2, 8])
def test_small_batch_n7(gpu, m):
    x, p, s = make_case(m, 256, 7, seed=7)
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M={m} N=7")


VALU_VARIANTS = [
    (rows, waves, unroll, cap)
    for rows in (1, 2, 4)
    for waves in (1, 4)
    for unroll in (1, 2, 4, 8)
    for cap in (0, 3)
    if not (rows == 4 and unroll == 8)
]
MFMA_VARIANTS = [(rows, splits, unroll, 0) for rows in (1, 2, 4) for splits in (1, 3, 8) for unroll in (1, 2, 4, 8)
                 if not (rows == 4 and unroll == 8)]


@pytest.mark.parametrize("kernel", [VALU, VOFF])
@pytest.mark.parametrize("rows,splits,unroll,cap", VALU_VARIANTS)
@pytest.mark.parametrize("k,n", [(256, 7), (1024, 13), (5632, 200), (14336, 40)])
def test_valu_variants_m1(gpu, kernel, rows, splits, unroll, cap, k, n):
    x, p, s = make_case(1, k, n, seed=3)
    out = _run_tuned(gpu, x, p, s, kernel, rows, splits, unroll, cap)
    assert_parity(out, expected(x, p, s), f"valu rows={rows} waves={splits} unroll={unroll} cap={cap}")


DIAG_VARIANTS = [
    (rows, waves, unroll, cap)
    for rows in (1, 2, 4)
    for waves in (1, 4)
    for unroll in (1, 2, 4)
    for cap in (0, 3)
    if not (rows == 4 and unroll == 4)
]


@pytest.mark.parametrize("rows,splits,unroll,cap", DIAG_VARIANTS)
@pytest.mark.parametrize("k,n", [(256, 7), (1024, 13), (5632, 200), (14336, 40), (2048, 64)])
def test_diag_variants_m1(gpu, rows, splits, unroll, cap, k, n):
    x, p, s = make_case(1, k, n, seed=5)
    out = _run_tuned(gpu, x, p, s, DIAG, rows, splits, unroll, cap)
    assert_parity(out, expected(x, p, s), f"diag rows={rows} waves={splits} unroll={unroll} cap={cap}")


@pytest.mark.parametrize("rows,splits,unroll,cap", MFMA_VARIANTS)
@pytest.mark.parametrize("k,n", [(256, 7), (1024, 13), (5632, 200)])
def test_mfma_variants_m1(gpu, rows, splits, unroll, cap, k, n):
    x, p, s = make_case(1, k, n, seed=3)
    out = _run_tuned(gpu, x, p, s, MFMA, rows, splits, unroll, cap)
    assert_parity(out, expected(x, p, s), f"mfma rows={rows} splits={splits} unroll={unroll}")


# K values: one partial load (256), whole loads (2048, 32768 = 16 loads), a
# ragged last load (5632: 176 chunks), 7 loads (14336) and 9 chunks-of-64
# rounded up to the 10-load instantiation (18432).
@pytest.mark.parametrize("rows,splits", [(1, 4), (2, 4), (1, 8), (2, 8)])
@pytest.mark.parametrize("k,n", [(256, 7), (2048, 13), (5632, 40), (14336, 21), (18432, 9), (32768, 5)])
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_oneshot_variants(gpu, m, rows, splits, k, n):
    x, p, s = make_case(m, k, n, seed=m * 31 + k + n)
    if m * k * 2 > 160 * 1024:
        with pytest.raises(_lib.W4A16Error, match="do not fit in LDS"):
            _run_tuned(gpu, x, p, s, ONESHOT, rows, splits, 0)
        return
    out = _run_tuned(gpu, x, p, s, ONESHOT, rows, splits, 0)
    assert_parity(out, expected(x, p, s), f"oneshot M={m} rows={rows} splits={splits} K={k} N={n}")


# 4 rows per wavefront (M = 1, 4 wavefronts): rows of one partial load up to
# 8 loads (16384), N not a multiple of 4 (the last wavefront's rows clamp)
@pytest.mark.parametrize("k,n", [(256, 7), (2048, 13), (2048, 2050), (5632, 41), (14336, 22), (16384, 9)])
def test_oneshot_four_rows(gpu, k, n):
    x, p, s = make_case(1, k, n, seed=k + n)
    out = _run_tuned(gpu, x, p, s, ONESHOT, 4, 4, 0)
    assert_parity(out, expected(x, p, s), f"oneshot rows=4 K={k} N={n}")


def test_oneshot_four_rows_all_nibbles_and_rejects(gpu):
    x, p, s = make_case(1, 1024, 66, seed=12, all_nibbles=True)
    assert_parity(_run_tuned(gpu, x, p, s, ONESHOT, 4, 4, 0), expected(x, p, s), "oneshot rows=4 all nibbles")
    x, p, s = make_case(1, 18432, 8, seed=13)   # 10 loads per row
    with pytest.raises(_lib.W4A16Error, match="rows 1 or 2"):
        _run_tuned(gpu, x, p, s, ONESHOT, 4, 4, 0)
    x, p, s = make_case(2, 2048, 8, seed=14)    # M = 2
    with pytest.raises(_lib.W4A16Error, match="rows 1 or 2"):
        _run_tuned(gpu, x, p, s, ONESHOT, 4, 4, 0)


# the M = 1 default on wide layers of short rows (the paired M = 1 kernel;
# 4 rows per wavefront of the one-shot kernel where K has no paired shape)
# and on 4096 x 4096, at full size
@pytest.mark.parametrize("k,n,kernel,rows,splits", [(2048, 32000, "pair_ring", 8, 1), (2048, 16384, "pair_ring", 8, 1),
                                                    (2048, 11264, "pair_ring", 3, 1), (4096, 4096, "pair_ring", 2, 2),
                                                    (1024, 24577, "oneshot", 4, 4), (2048, 2560, "oneshot", 1, 8)])
def test_default_dispatch_wide_m1(gpu, k, n, kernel, rows, splits):
    x, p, s = make_case(1, k, n, seed=k ^ n)
    plan = _lib.plan_linear(16, 16, 1, n, k)
    assert (plan["kernel"], plan["rows"], plan["splits"]) == (kernel, rows, splits)
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M=1 K={k} N={n} default")


# M = 2 through the default route on the ring kernel, the paired kernel (wide
# layers of short rows, rows above 6144 weights), the streaming paired kernel
# (wide layers of longer rows) and the one-shot kernel (rows of up to 6144),
# at full size
@pytest.mark.parametrize("k,n,kernel", [(2048, 32000, "mfma_pair"), (4096, 14336, "pair_ring"),
                                        (5632, 14336, "pair_stream"), (8192, 8192, "pair_ring"),
                                        (7168, 4096, "mfma_pair"), (6144, 4096, "oneshot"),
                                        (28672, 2048, "mfma_pair"), (11008, 28672, "pair_stream")])
def test_default_dispatch_m2(gpu, k, n, kernel):
    x, p, s = make_case(2, k, n, seed=k + 3 * n)
    assert _lib.plan_linear(16, 16, 2, n, k)["kernel"] == kernel
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M=2 K={k} N={n} default")


# one-shot MFMA: every (rows, splits) shape, K from one group to 32 groups
# (partial last step when splits do not divide K / 128), ragged N
@pytest.mark.parametrize("rows,splits", [(1, 4), (2, 4), (1, 8), (2, 8)])
@pytest.mark.parametrize("k,n", [(128, 7), (256, 40), (1152, 33), (2048, 2048), (3968, 21), (4096, 100),
                                 (4224, 9), (6144, 33), (8192, 64)])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 11, 16])
def test_mfma_oneshot_variants(gpu, m, rows, splits, k, n):
    if m * k * 2 + (k // 128) * 64 + splits * rows * 1024 > 160 * 1024:
        x, p, s = make_case(m, k, n, seed=1)
        with pytest.raises(_lib.W4A16Error, match="do not fit in LDS"):
            _run_tuned(gpu, x, p, s, MFMA_OS, rows, splits, 0)
        return
    x, p, s = make_case(m, k, n, seed=m * 13 + k + n)
    out = _run_tuned(gpu, x, p, s, MFMA_OS, rows, splits, 0)
    assert_parity(out, expected(x, p, s), f"mfma_oneshot M={m} rows={rows} splits={splits} K={k} N={n}")


def _pair_lds(m, staged, chunk, splits, blocks):
    slots = 4 if m <= 4 else 8 if m <= 8 else 16
    buffers = 2 if chunk < staged else 1
    return buffers * (chunk * 16 * 2 * slots * 16 + chunk * 128) + splits * blocks * 1024


# paired-group MFMA, whole rows staged (rows = splits * unroll): every
# (splits, blocks) class, odd group counts (a half pair zero-filled), splits *
# unroll past the last pair (padding pairs), ragged N, every row-slot width
# (M <= 4, M <= 8 and M = 9..16: one activation group per MFMA), K up to LDS
@pytest.mark.parametrize("splits,blocks", [(2, 1), (4, 2), (8, 1), (2, 8), (4, 4), (8, 2)])
@pytest.mark.parametrize("k,n", [(128, 7), (384, 9), (1152, 33), (2048, 2048), (3968, 21), (5632, 100),
                                 (8192, 64), (16384, 24)])
@pytest.mark.parametrize("m", [2, 3, 4, 6, 8])
def test_mfma_pair_whole(gpu, m, splits, blocks, k, n):
    pairs = (k // 128 + 1) // 2
    unroll = -(-pairs // splits)
    staged = splits * unroll
    if unroll > 8 or _pair_lds(m, staged, staged, splits, blocks) > 160 * 1024:
        x, p, s = make_case(m, k, n, seed=1)
        with pytest.raises(_lib.W4A16Error, match="no instantiation|do not fit in LDS"):
            _run_tuned(gpu, x, p, s, MFMA_PAIR, staged, splits, unroll, blocks)
        return
    x, p, s = make_case(m, k, n, seed=m * 17 + k + n)
    out = _run_tuned(gpu, x, p, s, MFMA_PAIR, staged, splits, unroll, blocks)
    assert_parity(out, expected(x, p, s), f"mfma_pair M={m} splits={splits} blocks={blocks} K={k} N={n}")


# 16 row slots (M = 9..16), whole rows: every (splits, blocks) class on rows
# up to 16 pairs (what LDS holds at 16 slots), odd group counts, padding
# pairs, ragged N
@pytest.mark.parametrize("splits,blocks", [(2, 1), (4, 2), (8, 1), (2, 8), (4, 4), (8, 2)])
@pytest.mark.parametrize("k,n", [(128, 7), (384, 9), (1152, 33), (2048, 2048), (3968, 21)])
@pytest.mark.parametrize("m", [9, 13, 16])
def test_mfma_pair_whole_16_slots(gpu, m, splits, blocks, k, n):
    pairs = (k // 128 + 1) // 2
    unroll = -(-pairs // splits)
    staged = splits * unroll
    assert _pair_lds(m, staged, staged, splits, blocks) <= 160 * 1024
    x, p, s = make_case(m, k, n, seed=m * 19 + k + n)
    out = _run_tuned(gpu, x, p, s, MFMA_PAIR, staged, splits, unroll, blocks)
    assert_parity(out, expected(x, p, s), f"mfma_pair 16 slots M={m} splits={splits} blocks={blocks} K={k} N={n}")


# chunked staging (rows = 8 pairs per chunk, two buffers): every
# instantiated (splits, blocks, unroll) class, odd group counts, padding
# pairs and a partial last chunk, rows up to K = 32768, ragged N
@pytest.mark.parametrize("splits,blocks,k", [(4, 1, 7168), (4, 4, 8192), (4, 2, 6400), (8, 1, 5632), (8, 2, 5760),
                                             (8, 1, 8192), (8, 2, 14336), (8, 1, 16512), (8, 2, 28672),
                                             (8, 1, 32768)])
@pytest.mark.parametrize("m", [2, 4, 5, 8, 12, 16])
def test_mfma_pair_chunked(gpu, m, splits, blocks, k):
    n = 37
    pairs = (k // 128 + 1) // 2
    unroll = -(-pairs // splits)
    if unroll > 8:
        unroll += unroll % 2
    assert _pair_lds(m, splits * unroll, 8, splits, blocks) <= 160 * 1024
    x, p, s = make_case(m, k, n, seed=m * 7 + k + blocks)
    # (M > 8 past 8 pairs per wavefront: no 16-slot kernel, two launches over the row halves)
    out = _run_tuned(gpu, x, p, s, MFMA_PAIR, 8, splits, unroll, blocks)
    assert_parity(out, expected(x, p, s), f"mfma_pair chunked M={m} splits={splits} blocks={blocks} K={k}")


@pytest.mark.parametrize("m,k,n", [(3, 2048, 9000), (5, 4352, 4096), (5, 5632, 2048), (7, 5632, 2560), (8, 8192, 1000),
                                   (4, 14336, 300), (6, 14336, 300), (8, 28672, 64), (3, 20480, 100),
                                   (5, 8320, 77),
                                   # M = 9..16 with the selector: one launch with 16 row slots, or two
                                   # over the row halves where that shape has no 16-slot kernel
                                   (16, 5632, 2048), (9, 28672, 100), (13, 8192, 77), (12, 2048, 11264)])
def test_default_dispatch_mfma_pair(gpu, m, k, n, monkeypatch):
    if m > 8:
        monkeypatch.setenv("W4A16_DECODE", "mfma_pair")   # M = 9..16 defaults to the GEMM
    x, p, s = make_case(m, k, n, seed=m + k + n)
    assert _lib.plan_linear(16, 16, m, n, k)["kernel"] == "mfma_pair"
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"pair default M={m} K={k} N={n}")


@pytest.mark.parametrize("rows", [0, 24, 8])
def test_mfma_pair_more_pairs_than_needed(gpu, rows):
    # splits * unroll = 24 pairs for the 2 of K = 512: padding pairs read
    # zeros and weigh 0, staged whole (24) or in chunks (8, and 0 = auto)
    x, p, s = make_case(5, 512, 40, seed=5)
    out = _run_tuned(gpu, x, p, s, MFMA_PAIR, rows, 8, 3, 1)
    assert_parity(out, expected(x, p, s), f"mfma_pair padded rows={rows}")


@pytest.mark.parametrize("m,k,splits", [(9, 2048, 4), (11, 2048, 4), (16, 2048, 4), (16, 20480, 8)])
def test_mfma_pair_m9_16_tuned(gpu, m, k, splits):
    # one launch with 16 row slots; rows past the 16-slot kernels (K = 20480:
    # 10 pairs per wavefront) run as two launches over the row halves
    x, p, s = make_case(m, k, 300, seed=m)
    out = _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, splits, 0, 2)
    assert_parity(out, expected(x, p, s), f"mfma_pair M={m} K={k}")


def test_mfma_pair_rejects(gpu):
    x, p, s = make_case(1, 2048, 8, seed=2)
    with pytest.raises(_lib.W4A16Error, match="2 <= M <= 16"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, 4, 0, 1)
    x, p, s = make_case(17, 2048, 8, seed=2)
    with pytest.raises(_lib.W4A16Error, match="2 <= M <= 16"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, 4, 0, 1)
    x, p, s = make_case(4, 2048, 8, seed=2)
    with pytest.raises(_lib.W4A16Error, match="cover the K / 256"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, 2, 1, 1)
    with pytest.raises(_lib.W4A16Error, match="splits 2, 4 or 8"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, 3, 0, 1)
    with pytest.raises(_lib.W4A16Error, match="no instantiation"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, 4, 0, 8)   # 32 wavefronts
    with pytest.raises(_lib.W4A16Error, match="no instantiation"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 2, 4, 0, 1)   # 2-pair chunks
    x, p, s = make_case(8, 8320, 8, seed=2)
    with pytest.raises(_lib.W4A16Error, match="do not fit in LDS"):
        _run_tuned(gpu, x, p, s, MFMA_PAIR, 40, 8, 5, 1)  # whole rows of 40 pairs


@pytest.mark.parametrize("depth", [2, 3, 4, 6])
@pytest.mark.parametrize("m", [2, 3, 5, 8])
@pytest.mark.parametrize("k,n", [(128, 7), (384, 100), (2048, 2048), (5632, 33), (8192, 40), (9216, 9)])
def test_pair_stream_variants(gpu, depth, m, k, n):
    """Streaming paired kernel: rows of 1 pair (fewer pairs than the ring),
    an odd group count (the last pair's second group zero-padded), ragged N,
    M of 2..8 (4 and 8 row slots) up to the longest rows that fit in LDS."""
    x, p, s = make_case(m, k, n, seed=m * 7 + k + n + depth)
    got = _run_tuned(gpu, x, p, s, PAIR_STREAM, 0, 1, depth)
    assert_parity(got, expected(x, p, s), f"pair_stream d={depth} M={m} K={k} N={n}")


@pytest.mark.parametrize("waves,cap", [(1, 1), (3, 2), (16, 1), (5, 7)])
@pytest.mark.parametrize("m,k,n", [(4, 2048, 300), (8, 1152, 97)])
def test_pair_stream_many_tasks(gpu, waves, cap, m, k, n):
    """Explicit wavefront counts and small grid caps: each wavefront streams
    many 8-row blocks, the ring crossing from one block's pairs to the next."""
    x, p, s = make_case(m, k, n, seed=waves * 11 + cap + m)
    got = _run_tuned(gpu, x, p, s, PAIR_STREAM, waves, 1, 3, max_blocks=cap)
    assert_parity(got, expected(x, p, s), f"pair_stream waves={waves} cap={cap} M={m} K={k} N={n}")


@pytest.mark.parametrize("m,k,n", [(3, 5632, 14343), (8, 8192, 28672), (5, 4224, 16384)])
def test_default_dispatch_pair_stream(gpu, m, k, n):
    """Wide layers route to the streaming paired kernel (ragged N, an odd
    group count at K = 4224)."""
    x, p, s = make_case(m, k, n, seed=m + k + n)
    assert _lib.plan_linear(1 << 20, 1 << 20, m, n, k, 128)["kernel"] == "pair_stream"
    assert_parity(_run_default(gpu, x, p, s, workspace=None), expected(x, p, s),
                  f"pair_stream default M={m} K={k} N={n}")


@pytest.mark.parametrize("depth", [2, 4, 6])
@pytest.mark.parametrize("m", [2, 3, 5, 8])
@pytest.mark.parametrize("k,n,splits", [(512, 7, 2), (1152, 100, 2), (1152, 33, 3), (2048, 2048, 4), (5504, 40, 11),
                                        (9216, 9, 5), (14336, 64, 7), (28672, 24, 16)])
def test_pair_split_variants(gpu, depth, m, k, n, splits):
    """Split-K streaming paired kernel: slices of one pair, a last slice
    shorter than the others and with an odd group count (K = 1152: 9 groups,
    slices of 3 + 2 pairs, or 2 + 2 + 1 with a last slice of one group; 5504
    over 11 slices: 2 pairs each, the last 3 groups), ragged N, M of 2..8, up
    to K = 28672 in 16 slices."""
    x, p, s = make_case(m, k, n, seed=m * 5 + k + n + depth + splits)
    got = _run_tuned(gpu, x, p, s, PAIR_SPLIT, 0, splits, depth)
    assert_parity(got, expected(x, p, s), f"pair_split d={depth} S={splits} M={m} K={k} N={n}")


@pytest.mark.parametrize("waves,cap", [(1, 1), (3, 2), (16, 1), (5, 7)])
@pytest.mark.parametrize("m,k,n,splits", [(4, 2048, 300, 2), (8, 1152, 97, 3), (8, 14336, 130, 4)])
def test_pair_split_many_tasks(gpu, waves, cap, m, k, n, splits):
    """Explicit wavefront counts and small caps on the workgroups per slice:
    each wavefront streams many 8-row blocks of its slice."""
    x, p, s = make_case(m, k, n, seed=waves * 13 + cap + m + splits)
    got = _run_tuned(gpu, x, p, s, PAIR_SPLIT, waves, splits, 3, max_blocks=cap)
    assert_parity(got, expected(x, p, s), f"pair_split waves={waves} cap={cap} S={splits} M={m} K={k} N={n}")


@pytest.mark.parametrize("m,k,n", [(8, 28672, 8192), (3, 28672, 8200), (5, 20480, 8192), (4, 16512, 8200)])
def test_default_dispatch_pair_split(gpu, m, k, n):
    """With a workspace, M = 3..8 layers with K > 16384 and N >= 8192 take the split-K
    kernel (the torch op's route; ragged N; K = 16512 has 129 groups, so the
    last of its 4 slices holds 27); without one, the same call takes the
    workspace-free route, also within the bar."""
    x, p, s = make_case(m, k, n, seed=m + k + n + 1)
    assert _lib.linear_workspace_bytes(m, n, k) > 0
    ref = expected(x, p, s)
    assert_parity(_run_default(gpu, x, p, s), ref, f"pair_split default M={m} K={k} N={n}")
    assert_parity(_run_default(gpu, x, p, s, workspace=None), ref, f"no workspace M={m} K={k} N={n}")


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_pair_split_unaligned_output(gpu, offset):
    """The reduce stores 4 outputs at a time only into an 8-byte aligned
    output; an output 2, 4 or 6 bytes past that (the C ABI asks for 2) takes
    the element-wise stores. M * N is a multiple of 4 here, and the elements
    around the output stay untouched."""
    m, k, n = 4, 20480, 8192
    x, p, s = make_case(m, k, n, seed=offset + 77)
    assert _lib.linear_workspace_bytes(m, n, k) > 0
    buf = torch.full((m * n + 8,), -7.0, dtype=torch.float16, device=gpu)
    out = buf[offset:offset + m * n].view(m, n)
    print(f"[case] pair_split output offset {2 * offset} B M={m} K={k} N={n}", flush=True)
    _lib.linear_f16(x.to(gpu), p.to(gpu), s.to(gpu), out)
    torch.cuda.synchronize()
    assert_parity(out, expected(x, p, s), f"pair_split offset {offset}")
    rest = torch.cat([buf[:offset], buf[offset + m * n:]]).cpu()
    assert torch.all(rest == -7.0)


def test_pair_split_workspace_reused(gpu):
    """Two calls in a row on one workspace (the second smaller), each against
    the oracle: partial sums of the first call do not leak into the second."""
    ws = torch.full((8 * 4096 * 16,), float("nan"), dtype=torch.float32, device=gpu)
    for m, k, n, splits in [(8, 14336, 4096, 14), (3, 2048, 1000, 2)]:
        x, p, s = make_case(m, k, n, seed=k + m)
        out = torch.full((m, n), float("nan"), dtype=torch.float16, device=gpu)
        print(f"[case] pair_split workspace reuse M={m} K={k} N={n} S={splits}", flush=True)
        _lib.linear_f16_tuned(x.to(gpu), p.to(gpu), s.to(gpu), out, 128, PAIR_SPLIT, 0, splits, 4, 0, workspace=ws)
        torch.cuda.synchronize()
        assert_parity(out, expected(x, p, s), f"pair_split reuse M={m} K={k} N={n}")


def test_pair_stream_rejects(gpu):
    x, p, s = make_case(8, 10240, 16, seed=4)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    out = torch.zeros((8, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="LDS"):   # 8 x 10240 activations do not fit
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, PAIR_STREAM, 0, 1, 2, 0)
    x, p, s = make_case(1, 2048, 16, seed=4)
    out1 = torch.zeros((1, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="2 <= M <= 8"):
        _lib.linear_f16_tuned(x.to(gpu), p.to(gpu), s.to(gpu), out1, 128, PAIR_STREAM, 0, 1, 2, 0)
    x, p, s = make_case(4, 2048, 16, seed=4)
    out4 = torch.zeros((4, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="unroll"):
        _lib.linear_f16_tuned(x.to(gpu), p.to(gpu), s.to(gpu), out4, 128, PAIR_STREAM, 0, 1, 5, 0)
    with pytest.raises(_lib.W4A16Error, match="wavefronts"):
        _lib.linear_f16_tuned(x.to(gpu), p.to(gpu), s.to(gpu), out4, 128, PAIR_STREAM, 17, 1, 2, 0)
    torch.cuda.synchronize()
    assert not out.any() and not out1.any() and not out4.any()


GEMM_SHAPES = [(1, 1, 2), (2, 1, 4), (4, 1, 8), (1, 2, 4), (2, 2, 8), (4, 2, 2), (1, 4, 8), (2, 4, 4), (4, 4, 2),
               (4, 4, 4)]


@pytest.mark.parametrize("rows,blocks,splits", GEMM_SHAPES)
@pytest.mark.parametrize("m,k,n", [(17, 2048, 200), (64, 384, 33), (100, 5632, 48), (3, 1152, 100)])
def test_gemm_variants(gpu, rows, blocks, splits, m, k, n):
    """The GEMM's instantiated tilings on ragged M and N (tiles past the
    end), K of 3..44 groups (wavefronts with no group when splits > K / 128)."""
    x, p, s = make_case(m, k, n, seed=m * 5 + k + n + rows)
    got = _run_tuned(gpu, x, p, s, GEMM, rows, splits, 0, max_blocks=blocks)
    assert_parity(got, expected(x, p, s), f"gemm {rows}/{blocks}/{splits} M={m} K={k} N={n}")


GEMM_LDS_SHAPES = [(2, 2, 2, 1), (2, 2, 2, 4), (2, 4, 2, 2), (2, 4, 4, 1), (4, 2, 2, 2), (4, 2, 4, 2), (4, 4, 2, 1),
                   (4, 4, 4, 2), (2, 2, 4, 4), (4, 2, 2, 4)]


@pytest.mark.parametrize("rows,blocks,sn,splits", GEMM_LDS_SHAPES)
@pytest.mark.parametrize("m,k,n", [(17, 2048, 200), (64, 384, 33), (100, 5632, 48), (3, 1152, 100), (70, 128, 300)])
def test_gemm_lds_variants(gpu, rows, blocks, sn, splits, m, k, n):
    """The LDS-staged GEMM's tilings on ragged M and N, K of 1..44 groups
    (rounds past the last group staged as zeros, rounds run to a multiple of
    the weight ring)."""
    x, p, s = make_case(m, k, n, seed=m * 3 + k + n + rows + sn)
    got = _run_tuned(gpu, x, p, s, GEMM_LDS, rows, splits, sn, max_blocks=blocks)
    assert_parity(got, expected(x, p, s), f"gemm_lds {rows}/{blocks}/{sn}/{splits} M={m} K={k} N={n}")


GEMM32_SHAPES = [(4, 2, 4, 1), (4, 1, 4, 1), (2, 1, 4, 2), (2, 2, 2, 2), (2, 2, 4, 1), (4, 1, 2, 2), (2, 1, 2, 4),
                 (2, 1, 1, 4)]


@pytest.mark.parametrize("rows,blocks,sn,splits", GEMM32_SHAPES)
@pytest.mark.parametrize("m,k,n", [(17, 2048, 200), (64, 384, 33), (100, 5632, 48), (3, 1152, 100), (70, 128, 300),
                                   (300, 4096, 700)])
def test_gemm32_variants(gpu, rows, blocks, sn, splits, m, k, n):
    """The 32x32-tile GEMM's tilings on ragged M and N, K of 1..44 groups
    (rounds past the last group staged as zeros; staging two rounds ahead
    runs past the end on clamped, never-read rounds)."""
    x, p, s = make_case(m, k, n, seed=m * 7 + k + n + rows + sn)
    got = _run_tuned(gpu, x, p, s, GEMM32, rows, splits, sn, max_blocks=blocks)
    assert_parity(got, expected(x, p, s), f"gemm32 {rows}/{blocks}/{sn}/{splits} M={m} K={k} N={n}")


def test_gemm32_rejects(gpu):
    x, p, s = make_case(64, 256, 64, seed=1)
    with pytest.raises(_lib.W4A16Error, match="32x32 GEMM kernel"):
        _run_tuned(gpu, x, p, s, GEMM32, 4, 2, 2, max_blocks=2)   # (4, 2, 2, 2): not instantiated


@pytest.mark.parametrize("m,k,n,kernel", [(17, 2048, 2048, "gemm"), (64, 2048, 5632, "gemm32"), (130, 5632, 2048, "gemm"),
                                          (512, 2048, 256, "gemm"), (33, 8192, 1000, "gemm"),
                                          (129, 4224, 4103, "gemm_lds"), (128, 4224, 4103, "gemm"), (200, 2048, 11300, "gemm32"),
                                          (256, 2048, 5632, "gemm32"), (128, 1024, 20480, "gemm32"),
                                          (100, 2048, 6000, "gemm32"), (64, 2048, 2048, "gemm"),
                                          (520, 1024, 8200, "gemm32"), (512, 4224, 4103, "gemm32")])
def test_default_dispatch_gemm(gpu, m, k, n, kernel):
    x, p, s = make_case(m, k, n, seed=m + k + 3 * n)
    assert _lib.plan_linear(1 << 20, 1 << 20, m, n, k, 128)["kernel"] == kernel
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"gemm default M={m} K={k} N={n}")


@pytest.mark.parametrize("m,k,n", [(48, 2048, 512), (200, 1024, 96)])
def test_gemm_uses_dequantized_weights(gpu, m, k, n):
    """The B operand is fp16_rn(code * scale), bit-identical to what
    w4a16_dequantize_f16 writes: against a float64 product of the activations
    with those dequantized weights the GEMM is within one fp16 rounding of the
    output (fp32 accumulation only reorders the sum)."""
    x, p, s = make_case(m, k, n, seed=m + n)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    wdq = torch.empty((n, k), dtype=torch.float16, device=gpu)
    _lib.dequantize_f16(pd, sd, wdq, 128)
    ref = (xd.double() @ wdq.double().t()).cpu()
    ulp = torch.finfo(torch.float16).eps / 2
    for kernel, rows, splits, unroll, blocks in ((GEMM, 4, 2, 0, 2), (GEMM_LDS, 4, 2, 2, 2), (GEMM32, 2, 2, 4, 1)):
        got = _run_tuned(gpu, x, p, s, kernel, rows, splits, unroll, max_blocks=blocks).double().cpu()
        assert torch.all((got - ref).abs() <= ulp * ref.abs() + 1e-4), (kernel, float((got - ref).abs().max()))


@pytest.mark.parametrize("m,k,n", [(16, 2048, 512), (12, 5632, 96)])
def test_mfma_pair_16_slots_uses_dequantized_weights(gpu, m, k, n):
    """16 row slots (M = 9..16): B is fp16_rn(code * scale), bit-identical to
    w4a16_dequantize_f16's weights, so the output is within one fp16
    rounding of a float64 product with them."""
    x, p, s = make_case(m, k, n, seed=m + n + 1)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    wdq = torch.empty((n, k), dtype=torch.float16, device=gpu)
    _lib.dequantize_f16(pd, sd, wdq, 128)
    ref = (xd.double() @ wdq.double().t()).cpu()
    ulp = torch.finfo(torch.float16).eps / 2
    got = _run_tuned(gpu, x, p, s, MFMA_PAIR, 0, 4 if k <= 4096 else 8, 0, 1).double().cpu()
    assert torch.all((got - ref).abs() <= ulp * ref.abs() + 1e-4), float((got - ref).abs().max())


def test_gemm_rejects(gpu):
    x, p, s = make_case(32, 2048, 16, seed=3)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    out = torch.zeros((32, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="splits"):
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, GEMM, 4, 8, 0, 4)   # 16 tiles with 8 wavefronts
    with pytest.raises(_lib.W4A16Error, match="rows"):
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, GEMM, 3, 4, 0, 1)
    with pytest.raises(_lib.W4A16Error, match="group_size 128"):
        _lib.linear_f16_tuned(xd, pd, sd, out, 64, GEMM, 2, 4, 0, 1)
    torch.cuda.synchronize()
    assert not out.any()


STREAM_SHAPES = [(2, 4, 2), (2, 8, 4), (4, 4, 3), (4, 8, 2), (4, 4, 4), (8, 4, 2), (8, 8, 2), (2, 4, 3),
                 (1, 4, 2), (1, 8, 4), (1, 8, 3)]


@pytest.mark.parametrize("rows,waves,depth", STREAM_SHAPES)
@pytest.mark.parametrize("k,n", [(128, 3), (2048, 7), (2176, 100), (8192, 7), (16384, 40), (16512, 9), (18432, 33),
                                 (28672, 21), (32768, 5)])
def test_stream_variants(gpu, rows, waves, depth, k, n):
    """Streaming kernel (M = 1): every instantiated shape on ragged rows
    (2176 = 1 step + 4 chunks, 16512 = 8 steps + 4 chunks), rows of fewer
    steps than the ring (128, 2048: the ring runs into the next rows, and
    wavefronts with fewer steps than the ring), both activation-unit counts
    (K <= 16384 and above) and N not a multiple of the rows per task."""
    x, p, s = make_case(1, k, n, seed=k + n + rows)
    got = _run_tuned(gpu, x, p, s, STREAM, rows, waves, depth)
    assert_parity(got, expected(x, p, s), f"stream {rows}/{waves}/{depth} K={k} N={n}")


@pytest.mark.parametrize("rows,waves,depth,cap", [(4, 4, 3, 1), (2, 8, 4, 3), (8, 4, 2, 2), (4, 8, 2, 5)])
@pytest.mark.parametrize("k,n", [(2048, 203), (8192, 203), (16512, 77)])
def test_stream_many_tasks_per_wavefront(gpu, rows, waves, depth, cap, k, n):
    """A small grid cap gives each wavefront many tasks, so the ring of
    in-flight steps crosses from one task's rows to the next (and the
    peeled tail starts inside a task)."""
    x, p, s = make_case(1, k, n, seed=k * 3 + n + cap)
    got = _run_tuned(gpu, x, p, s, STREAM, rows, waves, depth, max_blocks=cap)
    assert_parity(got, expected(x, p, s), f"stream cap {cap} {rows}/{waves}/{depth} K={k} N={n}")


@pytest.mark.parametrize("k,n", [(16384, 64), (28672, 100), (32768, 33)])
def test_default_dispatch_long_rows_m1(gpu, k, n):
    x, p, s = make_case(1, k, n, seed=k + 2 * n)
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M=1 K={k} N={n}")


def test_stream_rejects(gpu):
    x, p, s = make_case(2, 4096, 16, seed=5)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    out = torch.zeros((2, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="M == 1"):
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, STREAM, 4, 4, 2, 0)
    out1 = torch.zeros((1, 16), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="rows 1, 2 or 4"):
        _lib.linear_f16_tuned(xd[:1], pd, sd, out1, 128, STREAM, 3, 4, 3, 0)
    with pytest.raises(_lib.W4A16Error, match="rows 8 with unroll 2"):
        _lib.linear_f16_tuned(xd[:1], pd, sd, out1, 128, STREAM, 8, 4, 3, 0)
    with pytest.raises(_lib.W4A16Error, match="splits"):
        _lib.linear_f16_tuned(xd[:1], pd, sd, out1, 128, STREAM, 4, 2, 2, 0)
    torch.cuda.synchronize()
    assert not out.any() and not out1.any()


@pytest.mark.parametrize("kernel", ["default", "mfma_oneshot"])
@pytest.mark.parametrize("m,k,n,default", [(9, 2048, 300, "gemm"), (16, 2048, 2048, "pair_ring"),
                                           (16, 4096, 64, "gemm"), (12, 256, 7, "gemm"),
                                           (16, 5632, 2048, "mfma_pair"), (16, 2048, 2560, "pair_ring"),
                                           (11, 5632, 2048, "mfma_pair"), (16, 4096, 14336, "gemm"),
                                           (12, 2048, 11264, "pair_ring"), (9, 14336, 4096, "mfma_pair"),
                                           (16, 8192, 8192, "gemm"), (12, 2048, 32000, "gemm")])
def test_default_dispatch_short_prompt(gpu, m, k, n, default, kernel, monkeypatch):
    """M = 9..16 without a workspace: the paired ring kernel's 16-row-slot
    form on rows of 2048 weights of 1024 .. 16384-row layers, the paired
    kernel in one launch (16 row slots) on rows longer than 4096 weights (at
    most 256 workgroups and 2 wavefronts on weight blocks), else the GEMM;
    the one-shot MFMA kernel with its selector (where its activations fit in
    LDS). The run itself goes through the op's route with a workspace (K
    slices of the ring kernel at M >= 12 on 5632 x 2048, 14336 x 4096 and
    8192 x 8192)."""
    if kernel == "mfma_oneshot":
        if m * k * 2 > 100 * 1024:
            pytest.skip("activations past the one-shot MFMA kernel's LDS")
        monkeypatch.setenv("W4A16_DECODE", "mfma_oneshot")
    else:
        kernel = default
    x, p, s = make_case(m, k, n, seed=m + k)
    assert _lib.plan_linear(16, 16, m, n, k)["kernel"] == kernel
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"prompt M={m} K={k} N={n} {kernel}")


def test_mfma_oneshot_rejects(gpu):
    x, p, s = make_case(2, 8320, 8, seed=2)
    with pytest.raises(_lib.W4A16Error, match="up to 8192"):
        _run_tuned(gpu, x, p, s, MFMA_OS, 1, 4, 0)
    x, p, s = make_case(2, 2048, 8, seed=2)
    with pytest.raises(_lib.W4A16Error, match="cover K"):
        _run_tuned(gpu, x, p, s, MFMA_OS, 1, 4, 2)
    with pytest.raises(_lib.W4A16Error, match="splits must be 4 or 8"):
        _run_tuned(gpu, x, p, s, MFMA_OS, 1, 2, 0)


@pytest.mark.parametrize("unroll", [2, 4, 8, 16])
def test_oneshot_more_loads_than_needed(gpu, unroll):
    # lanes past the row's last chunk idle on every extra load
    x, p, s = make_case(1, 1024, 33, seed=unroll)
    out = _run_tuned(gpu, x, p, s, ONESHOT, 1, 4, unroll)
    assert_parity(out, expected(x, p, s), f"oneshot unroll={unroll}")


def test_oneshot_rejects_short_unroll_and_long_rows(gpu):
    x, p, s = make_case(1, 4096, 8, seed=3)
    with pytest.raises(_lib.W4A16Error, match="too small"):
        _run_tuned(gpu, x, p, s, ONESHOT, 1, 4, 1)
    with pytest.raises(_lib.W4A16Error, match="rows 1 or 2"):
        _run_tuned(gpu, x, p, s, ONESHOT, 4, 8, 0)   # 4 rows run with 4 wavefronts only
    x, p, s = make_case(1, 34816, 3, seed=4)
    with pytest.raises(_lib.W4A16Error, match="K > 32768"):
        _run_tuned(gpu, x, p, s, ONESHOT, 1, 8, 0)
    # the default plan falls back to the looped VALU kernel for such rows
    plan = _lib.plan_linear(16, 16, 1, 3, 34816)
    assert plan["kernel"] == "valu"
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), "M=1 K=34816 default")


@pytest.mark.parametrize("kernel,rows,splits,unroll,cap",
                         [(ONESHOT, 1, 4, 0, 0), (ONESHOT, 2, 8, 0, 0), (MFMA_OS, 2, 4, 0, 0), (MFMA_OS, 1, 8, 0, 0),
                          (VALU, 1, 1, 1, 0), (VALU, 2, 4, 2, 0), (VALU, 4, 2, 1, 5), (VALU, 2, 4, 8, 0),
                          (VOFF, 1, 1, 1, 0), (VOFF, 2, 4, 2, 0), (VOFF, 4, 2, 1, 5), (VOFF, 2, 4, 8, 0),
                          (MFMA, 1, 1, 1, 0), (MFMA, 2, 4, 2, 0), (MFMA, 4, 2, 1, 0)])
@pytest.mark.parametrize("m", [1, 2, 5, 8])
def test_tuned_variants_batch(gpu, kernel, rows, splits, unroll, cap, m):
    x, p, s = make_case(m, 2048, 300, seed=m)
    if kernel == VOFF and m != 1:
        with pytest.raises(_lib.W4A16Error, match="M == 1 only"):
            _run_tuned(gpu, x, p, s, kernel, rows, splits, unroll, cap)
        return
    if kernel == ONESHOT and m > 4:
        with pytest.raises(_lib.W4A16Error, match="1 <= M <= 4"):
            _run_tuned(gpu, x, p, s, kernel, rows, splits, unroll, cap)
        return
    out = _run_tuned(gpu, x, p, s, kernel, rows, splits, unroll, cap)
    assert_parity(out, expected(x, p, s), f"kernel={kernel} M={m}")


@pytest.mark.parametrize("kernel", [VALU, VOFF, ONESHOT, MFMA, MFMA_OS, GENERIC, DIAG, STREAM])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_all_nibble_values(gpu, kernel, m):
    if kernel in (DIAG, VOFF, STREAM) and m != 1:
        pytest.skip("the diagonal MFMA, offset-decode VALU and streaming kernels are M = 1 only")
    if kernel == ONESHOT and m > 4:
        pytest.skip("the one-shot kernel is built for M <= 4")
    # random bytes: all 16 codes (incl. -8) in both nibbles of every byte position
    x, p, s = make_case(m, 1024, 64, seed=11, all_nibbles=True)
    if kernel in (ONESHOT, MFMA_OS):
        out = _run_tuned(gpu, x, p, s, kernel, 2, 4, 0)
    elif kernel == STREAM:
        x, p, s = make_case(m, 4096, 64, seed=11, all_nibbles=True)   # two steps of 1 KiB per row
        out = _run_tuned(gpu, x, p, s, kernel, 4, 4, 2)
    else:
        out = _run_tuned(gpu, x, p, s, kernel, 2, 2, 2)
    assert_parity(out, expected(x, p, s), f"all nibbles kernel={kernel} M={m}")


def _stress_activations(kind: str, m: int, k: int) -> torch.Tensor:
    gen = torch.Generator().manual_seed(17)
    if kind == "constant":        # every group sum large and one-signed
        return torch.full((m, k), 60.0).to(torch.float16)
    if kind == "outliers":        # N(0,1) with 1% channels at +-300
        x = torch.randn((m, k), generator=gen)
        idx = torch.randperm(k, generator=gen)[: k // 100]
        x[:, idx] = 300.0 * torch.sign(torch.randn((m, idx.numel()), generator=gen))
        return x.to(torch.float16)
    if kind == "cancel":          # +c then -c within each group: sum x per group = 0, sum |x| large
        x = torch.full((m, k), 40.0)
        x[:, 1::2] = -40.0
        return x.to(torch.float16)
    raise ValueError(kind)


@pytest.mark.parametrize("kernel,rows,splits,unroll", [(VALU, 2, 4, 1), (VOFF, 2, 4, 1), (VOFF, 1, 4, 8),
                                                       (ONESHOT, 2, 4, 0), (ONESHOT, 1, 8, 0),
                                                       (MFMA_OS, 1, 4, 0), (MFMA_OS, 2, 8, 0),
                                                       (DIAG, 2, 4, 1), (DIAG, 1, 4, 2),
                                                       (MFMA, 2, 4, 1), (GENERIC, 1, 1, 1), (STREAM, 4, 4, 2)])
@pytest.mark.parametrize("kind", ["constant", "outliers", "cancel"])
def test_precision_stress(gpu, kernel, rows, splits, unroll, kind):
    m = 1 if kernel in (DIAG, VOFF, STREAM) else 4
    _, p, s = make_case(m, 4096, 96, seed=21)
    x = _stress_activations(kind, m, 4096)
    out = _run_tuned(gpu, x, p, s, kernel, rows, splits, unroll)
    assert_parity(out, expected(x, p, s), f"stress {kind} kernel={kernel}")


@pytest.mark.parametrize("m", [1, 3, 9, 16])
@pytest.mark.parametrize("group_size", [32, 64, 128, 6])
def test_generic_kernel_any_group(gpu, m, group_size):
    k = 384 if group_size != 6 else 396
    x, p, s = make_case(m, k, 19, seed=group_size, group_size=group_size)
    out = _run_default(gpu, x, p, s, group_size)
    assert_parity(out, expected(x, p, s, group_size), f"generic M={m} G={group_size}")


def test_misaligned_activations_take_generic(gpu):
    x, p, s = make_case(1, 2048, 96, seed=5)
    buf = torch.empty(2048 + 1, dtype=torch.float16, device=gpu)
    buf[1:] = x.to(gpu)[0]
    xd = buf[1:].view(1, 2048)
    assert xd.data_ptr() % 16 != 0
    plan = _lib.plan_linear(xd.data_ptr(), 0, 1, 96, 2048)
    assert plan["kernel"] == "generic"
    out = torch.empty((1, 96), dtype=torch.float16, device=gpu)
    _lib.linear_f16(xd, p.to(gpu), s.to(gpu), out)
    torch.cuda.synchronize()
    assert_parity(out, expected(x, p, s), "misaligned")


@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 14336), (14336, 4096), (8192, 8192), (8192, 28672),
                                 (28672, 8192)])
@pytest.mark.parametrize("m", [1, 8])
def test_large_shapes(gpu, k, n, m):
    x, p, s = make_case(m, k, n, seed=1, device="cuda")
    assert_parity(_run_default(gpu, x, p, s), expected(x, p, s), f"M={m} K={k} N={n}")


@pytest.mark.parametrize("group_size", [32, 64, 128])
@pytest.mark.parametrize("k,n", [(256, 8), (2048, 2048), (2048, 5632), (5632, 2048)])
def test_dequantize_bit_identical(gpu, group_size, k, n):
    _, p, s = make_case(1, k, n, seed=k, group_size=group_size)
    out = torch.empty((n, k), dtype=torch.float16, device=gpu)
    _lib.dequantize_f16(p.to(gpu), s.to(gpu), out, group_size)
    torch.cuda.synchronize()
    ref = oracle.dequantize_f16(p.numpy(), s.numpy(), group_size)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_dequantize_all_codes_all_finite_scales(gpu):
    # every finite fp16 scale bit pattern (incl. subnormals, +-0) x all 16 codes;
    # products overflow to inf for large scales and land on fp16 subnormals for
    # tiny ones
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = bits[np.isfinite(bits.view(np.float16))]
    n = finite.size                      # 63490 rows of one 32-wide group
    codes_row = np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE] * 2, dtype=np.uint8)
    packed = np.tile(codes_row, (n, 1))  # K = 32: codes 0,1,..,7,-8,..,-1 twice
    scales = finite.view(np.float16).reshape(n, 1)
    out = torch.empty((n, 32), dtype=torch.float16, device=gpu)
    _lib.dequantize_f16(torch.from_numpy(packed).to(gpu), torch.from_numpy(scales.copy()).to(gpu), out, 32)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    ref = oracle.dequantize_f16(packed, scales, 32).view(np.uint16)
    # NaN payloads are not part of the contract; scales here are finite, so
    # 0 * finite never makes NaN
    assert np.array_equal(got, ref)
