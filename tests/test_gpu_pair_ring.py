"""GPU parity of the paired-layout M = 1 kernel (w4a16_pair_m1.h) against the
CPU oracle, through the C ABI: every instantiated launch shape (tuned entry
point), ragged N, K with a shorter last slice, all sixteen nibble codes, the
default route at full size on every configs shape it takes, the fallback
for 4-byte misaligned scales, and its rejects. Bar: |err| <= 1e-2 (1 + |ref|)."""

from __future__ import annotations

import pytest
import torch

import oracle
from nibble_amd import _lib
from tests._cases import assert_parity, expected, make_case

pytestmark = pytest.mark.gpu

RING = _lib.KERNEL_PAIR_RING

# (splits = wavefronts splitting K, rows = 8-row-block wavefronts, unroll =
# pairs in flight, K values whose pairs per wavefront match the instantiation)
SHAPES = [
    (1, 3, 8, (2048,)),
    (1, 3, 7, (2048,)),
    (1, 3, 6, (2048,)),
    (1, 8, 4, (2048,)),
    (2, 2, 8, (4096, 3840)),            # 3840: 15 pairs, the second slice one short
    (2, 2, 7, (4096, 3840)),
    (1, 8, 6, (4096,)),
    (4, 1, 6, (6144, 5632, 5376)),      # 5632: 22 pairs over 4 slices of 6
    (2, 4, 4, (8192, 7936)),
    (2, 4, 6, (8192, 7936)),
    (1, 7, 6, (8192,)),
    (2, 2, 10, (14336, 14080)),
    (2, 4, 6, (28672, 28416)),
]
VARIANTS = [(sk, sn, d, k) for sk, sn, d, ks in SHAPES for k in ks]

# M = 2..4 (4 row slots) and M = 5..8 (8 row slots)
SHAPES4 = [(4, 1, 2, (2048, 1792)), (1, 4, 6, (2048,)), (1, 4, 7, (2048,)), (2, 2, 4, (4096, 3840)),
           (2, 2, 6, (4096, 3840)), (1, 8, 6, (4096,)),
           (8, 1, 3, (5632, 6144)), (2, 4, 4, (8192,)), (4, 2, 6, (14336, 14080))]
SHAPES8 = [(4, 1, 2, (2048,)), (1, 4, 6, (2048,)), (4, 2, 4, (4096, 3840)), (1, 8, 6, (4096,)), (2, 4, 4, (8192, 7936)),
           (2, 4, 5, (8192, 7936)),
           (11, 1, 2, (5632, 5376))]   # 5376: 21 pairs, the last wavefront one short
SMALL = ([(m, sk, sn, d, k) for sk, sn, d, ks in SHAPES4 for k in ks for m in (2, 3, 4)] +
         [(m, sk, sn, d, k) for sk, sn, d, ks in SHAPES8 for k in ks for m in (5, 8)])


# M = 9..16 (16 row slots, exact decode): (splits, rows, unroll, K slices,
# K values whose pairs per wavefront per slice match the instantiation)
SHAPES16 = [(8, 1, 1, 1, (2048, 1792)), (4, 2, 2, 1, (2048, 1536)), (2, 4, 4, 1, (2048, 1792)),
            (1, 4, 4, 1, (2048,)),
            (1, 8, 3, 8, (5632, 6144)),      # 5632: 22 pairs in 8 slices of 3, the last holding 1
            (1, 8, 4, 4, (14336, 14080)), (1, 8, 4, 2, (8192, 7936))]   # 14 / 16 pairs per wavefront
PROMPT = [(m, sk, sn, d, sl, k) for sk, sn, d, sl, ks in SHAPES16 for k in ks for m in (9, 13, 16)]
# M = 2..4 with K slices: 28672 (112 pairs) and 28416 (111: the last slice one short) in 4 slices of 28
SLICED4 = [(m, 1, 8, 4, 4, k) for k in (28672, 28416) for m in (2, 3, 4)]
# M = 5..8 with K slices and two 8-row blocks per wavefront: 8 slices of 14 pairs (28672, 28416) and 2 of 16
# (8192, 7936)
SLICED8 = ([(m, 1, 8, 2, 8, k) for k in (28672, 28416) for m in (5, 8)] +
           [(m, 1, 8, 3, 2, k) for k in (8192, 7936) for m in (5, 8)])


def _run(dev, x, p, s, kernel=None, rows=0, splits=0, unroll=0, slices=0):
    xd, pd, sd = x.to(dev), p.to(dev), s.to(dev)
    out = torch.full((x.shape[0], p.shape[0]), float("nan"), dtype=torch.float16, device=dev)
    print(f"[case] kernel={kernel} rows={rows} splits={splits} unroll={unroll} slices={slices} M={x.shape[0]} "
          f"K={x.shape[1]} N={p.shape[0]}", flush=True)
    if kernel is None:
        _lib.linear_f16(xd, pd, sd, out)
    else:
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, kernel, rows, splits, unroll, slices)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("splits,rows,unroll,k", VARIANTS)
@pytest.mark.parametrize("n", [7, 65, 300])
def test_pair_ring_m1_variants(gpu, splits, rows, unroll, k, n):
    """Every instantiated shape on ragged N (partial 8-row blocks, a partial
    last workgroup), against the oracle."""
    x, p, s = make_case(1, k, n, seed=k + 7 * n + splits)
    out = _run(gpu, x, p, s, RING, rows, splits, unroll)
    assert_parity(out, expected(x, p, s), f"pair_m1 ({splits},{rows},{unroll}) K={k} N={n}")


@pytest.mark.parametrize("m,splits,rows,unroll,k", SMALL)
@pytest.mark.parametrize("n", [13, 300])
def test_pair_ring_small_batch_variants(gpu, m, splits, rows, unroll, k, n):
    """Every M = 2..8 shape at every M of its row slots (rows past M in the
    A operand and in the stores), ragged N, against the oracle."""
    x, p, s = make_case(m, k, n, seed=k + 5 * n + 11 * m + splits)
    out = _run(gpu, x, p, s, RING, rows, splits, unroll)
    assert_parity(out, expected(x, p, s), f"pair_ring M={m} ({splits},{rows},{unroll}) K={k} N={n}")


@pytest.mark.parametrize("m,splits,rows,unroll,k", [(1, 2, 2, 8, 4096), (1, 4, 1, 6, 5632), (1, 2, 2, 10, 14336),
                                                    (3, 8, 1, 3, 5632), (8, 4, 2, 4, 4096), (8, 2, 4, 4, 8192)])
def test_pair_ring_m1_all_nibbles(gpu, m, splits, rows, unroll, k):
    """Uniform random bytes (code -8 included) with scales in [0.01, 1.01)."""
    x, p, s = make_case(m, k, 97, seed=5, all_nibbles=True)
    out = _run(gpu, x, p, s, RING, rows, splits, unroll)
    assert_parity(out, expected(x, p, s), f"pair_m1 all nibbles K={k}")


# every configs shape the default M = 1 route sends to this kernel, at full
# size (configs[1], [2] at M = 1, [3], and the 1.1B model's lm_head)
@pytest.mark.parametrize("k,n", [(2048, 5632), (5632, 2048), (4096, 4096), (4096, 14336), (14336, 4096),
                                 (8192, 8192), (8192, 28672), (28672, 8192), (2048, 32000)])
def test_pair_ring_m1_default_route_full_size(gpu, k, n):
    """M = 1 through the default route (the plan the benchmark times)."""
    x, p, s = make_case(1, k, n, seed=k ^ (3 * n), device="cuda")
    assert _lib.plan_linear(16, 16, 1, n, k)["kernel"] == "pair_ring"
    assert_parity(_run(gpu, x, p, s), expected(x, p, s), f"M=1 K={k} N={n} default (pair_m1)")


# the M = 2..8 configs[2] / configs[3] shapes the default route sends here
@pytest.mark.parametrize("m,k,n", [(2, 2048, 2048), (4, 2048, 5632), (8, 2048, 5632), (8, 2048, 2048),
                                   (2, 4096, 4096), (8, 4096, 4096), (2, 4096, 14336), (4, 4096, 14336),
                                   (8, 4096, 14336), (4, 8192, 8192), (8, 8192, 8192), (2, 14336, 4096),
                                   (4, 14336, 4096), (4, 5632, 2048), (6, 5632, 2048), (8, 5632, 2048)])
def test_pair_ring_default_route_small_batch_full_size(gpu, m, k, n):
    x, p, s = make_case(m, k, n, seed=m + k ^ (5 * n), device="cuda")
    assert _lib.plan_linear(16, 16, m, n, k)["kernel"] == "pair_ring"
    assert_parity(_run(gpu, x, p, s), expected(x, p, s), f"M={m} K={k} N={n} default (pair_ring)")


def test_pair_ring_m1_misaligned_scales_fall_back(gpu):
    """Scales 2-byte but not 4-byte aligned: the default route takes another
    kernel (this one reads scale pairs as 32-bit words), the tuned entry
    point rejects it."""
    k, n = 4096, 14336
    x, p, s = make_case(1, k, n, seed=21, device="cuda")
    xd, pd = x.to(gpu), p.to(gpu)
    buf = torch.empty(s.numel() + 1, dtype=torch.float16, device=gpu)
    sd = buf[1:].view(n, k // 128)
    sd.copy_(s.to(gpu))
    assert sd.data_ptr() % 4 == 2
    out = torch.full((1, n), float("nan"), dtype=torch.float16, device=gpu)
    _lib.linear_f16(xd, pd, sd, out)
    torch.cuda.synchronize()
    assert_parity(out, expected(x, p, s), "misaligned scales, default route")
    with pytest.raises(_lib.W4A16Error, match="4-byte aligned"):
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, RING, 8, 1, 6)


def test_pair_ring_m1_rejects(gpu):
    x, p, s = make_case(1, 2176, 16, seed=3)   # 17 groups: K not a multiple of 256
    with pytest.raises(_lib.W4A16Error, match="multiple of 256"):
        _run(gpu, x, p, s, RING, 3, 1, 8)
    x, p, s = make_case(1, 4096, 16, seed=3)
    with pytest.raises(_lib.W4A16Error, match="not instantiated"):
        _run(gpu, x, p, s, RING, 3, 1, 8)     # 16 pairs per wavefront with 3 row wavefronts: no such shape
    x, p, s = make_case(2, 2048, 16, seed=3)
    with pytest.raises(_lib.W4A16Error, match="not instantiated for this M"):
        _run(gpu, x, p, s, RING, 3, 1, 8)     # an M = 1 shape
    x, p, s = make_case(9, 4096, 16, seed=3)
    with pytest.raises(_lib.W4A16Error, match="not instantiated for this M"):
        _run(gpu, x, p, s, RING, 8, 1, 6)     # an M = 1..8 shape at M = 9
    x, p, s = make_case(17, 2048, 16, seed=3)
    with pytest.raises(_lib.W4A16Error, match="1 <= M <= 16"):
        _run(gpu, x, p, s, RING, 1, 8, 1)
    x, p, s = make_case(16, 5632, 16, seed=3)
    with pytest.raises(_lib.W4A16Error, match="each slice non-empty"):
        _run(gpu, x, p, s, RING, 8, 1, 3, slices=12)   # 22 pairs in 12 slices of 2: the last empty
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    out = torch.empty((16, 16), dtype=torch.float16, device=gpu)
    small = torch.empty((16 * 16 * 8 - 1,), dtype=torch.float32, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="workspace"):
        _lib.linear_f16_tuned(xd, pd, sd, out, 128, RING, 8, 1, 3, 8, workspace=small)


@pytest.mark.parametrize("m,splits,rows,unroll,slices,k", PROMPT)
@pytest.mark.parametrize("n", [13, 300])
def test_pair_ring_prompt_variants(gpu, m, splits, rows, unroll, slices, k, n):
    """Every M = 9..16 shape (16 row slots, K slices included) at M = 9, 13
    and 16, ragged N, K with a short or padded last slice, against the
    oracle."""
    x, p, s = make_case(m, k, n, seed=k + 3 * n + 13 * m + splits)
    out = _run(gpu, x, p, s, RING, rows, splits, unroll, slices)
    assert_parity(out, expected(x, p, s), f"pair_ring M={m} ({splits},{rows},{unroll}) x{slices} K={k} N={n}")


@pytest.mark.parametrize("splits,rows,unroll,slices,k", [(sk, sn, d, sl, ks[0]) for sk, sn, d, sl, ks in SHAPES16])
def test_pair_ring_prompt_uses_dequantized_weights(gpu, splits, rows, unroll, slices, k):
    """16 row slots: B is fp16_rn(code * scale), w4a16_dequantize_f16's
    weights, summed in fp32: the reference's prefill path (dequantize, fp16
    GEMM). With four nonzero activations per row (small integers and halves)
    every product and partial sum is exact in fp32, so the output must equal
    the float64 product with the dequantized weights rounded to fp16, bit for
    bit; scaling exact codes in fp32 instead (the M <= 8 decode) would miss it
    wherever code * scale is not an fp16 value."""
    m, n = 16, 96
    x, p, s = make_case(m, k, n, seed=k + splits, all_nibbles=True)
    gen = torch.Generator().manual_seed(k)
    x = torch.zeros((m, k), dtype=torch.float16)
    vals = torch.tensor([-3.0, -2.0, -1.0, -0.5, 0.5, 1.0, 2.0, 3.0], dtype=torch.float16)
    for r in range(m):
        cols = torch.randperm(k, generator=gen)[:4]
        x[r, cols] = vals[torch.randint(0, 8, (4,), generator=gen)]
    pd, sd = p.to(gpu), s.to(gpu)
    wdq = torch.empty((n, k), dtype=torch.float16, device=gpu)
    _lib.dequantize_f16(pd, sd, wdq, 128)
    ref = (x.to(gpu).double() @ wdq.double().t()).to(torch.float16).cpu()
    got = _run(gpu, x, p, s, RING, rows, splits, unroll, slices).cpu()
    assert torch.equal(got, ref), int((got != ref).sum())
    # the check discriminates: exact codes times the scale, unrounded (the
    # M <= 8 decode's sums), land on other fp16 values for some outputs
    q = torch.from_numpy(oracle.unpack_int4(p.numpy())).double()
    alt = (x.double() @ (q * s.double().repeat_interleave(128, dim=1)).t()).to(torch.float16)
    assert not torch.equal(alt, ref)


# the 1.1B model's prompt projections (M = 16, and M = 9 / 12 at the slice
# threshold) through the default route with a workspace, as the op runs them
@pytest.mark.parametrize("m,k,n,slices", [(16, 2048, 2048, 0), (16, 2048, 2560, 0), (16, 2048, 11264, 0),
                                          (9, 2048, 2560, 0), (16, 5632, 2048, 8), (12, 5632, 2048, 8),
                                          (16, 14336, 4096, 4), (16, 8192, 8192, 2)])
def test_pair_ring_prompt_default_route(gpu, m, k, n, slices):
    x, p, s = make_case(m, k, n, seed=m + k ^ (7 * n), device="cuda")
    if slices == 0:
        assert _lib.plan_linear(16, 16, m, n, k)["kernel"] == "pair_ring"
    assert _lib.linear_workspace_bytes(m, n, k) == slices * m * n * 4
    assert_parity(_run(gpu, x, p, s), expected(x, p, s), f"M={m} K={k} N={n} default (pair_ring, {slices} slices)")


@pytest.mark.parametrize("m,splits,rows,unroll,slices,k", SLICED4)
@pytest.mark.parametrize("n", [13, 300])
def test_pair_ring_sliced_small_batch_variants(gpu, m, splits, rows, unroll, slices, k, n):
    """4 row slots over K slices (the workspace route of M = 3..4 on rows of
    28672), every M of the slots, ragged N, a short last slice, against the
    oracle."""
    x, p, s = make_case(m, k, n, seed=k + 3 * n + 17 * m)
    out = _run(gpu, x, p, s, RING, rows, splits, unroll, slices)
    assert_parity(out, expected(x, p, s), f"pair_ring M={m} x{slices} K={k} N={n}")


@pytest.mark.parametrize("m", [3, 4])
def test_pair_ring_sliced_default_route_full_size(gpu, m):
    """28672 x 8192 at M = 3..4 through the default route with a workspace
    (4 K slices of the ring kernel), as the op runs it."""
    k, n = 28672, 8192
    x, p, s = make_case(m, k, n, seed=m + 5, device="cuda")
    assert _lib.linear_workspace_bytes(m, n, k) == 4 * m * n * 4
    assert_parity(_run(gpu, x, p, s), expected(x, p, s), f"M={m} K={k} N={n} default (ring, 4 K slices)")


@pytest.mark.parametrize("m,splits,rows,unroll,slices,k", SLICED8)
@pytest.mark.parametrize("n", [13, 300])
def test_pair_ring_sliced_two_blocks_variants(gpu, m, splits, rows, unroll, slices, k, n):
    """8 row slots over K slices with two 8-row blocks per wavefront (a
    workgroup covers 128 rows: ragged N leaves most of it past N), against
    the oracle."""
    x, p, s = make_case(m, k, n, seed=k + 7 * n + 19 * m)
    out = _run(gpu, x, p, s, RING, rows, splits, unroll, slices)
    assert_parity(out, expected(x, p, s), f"pair_ring RB2 M={m} x{slices} K={k} N={n}")


@pytest.mark.parametrize("m,k,n,slices", [(5, 28672, 8192, 8), (8, 28672, 8192, 8), (6, 8192, 28672, 2),
                                          (8, 8192, 28672, 2)])
def test_pair_ring_sliced_two_blocks_default_route(gpu, m, k, n, slices):
    """The 70B-class layers at M = 5..8 through the default route with a
    workspace, as the op runs them."""
    x, p, s = make_case(m, k, n, seed=m + k + n, device="cuda")
    assert _lib.linear_workspace_bytes(m, n, k) == slices * m * n * 4
    assert_parity(_run(gpu, x, p, s), expected(x, p, s), f"M={m} K={k} N={n} default (ring RB2, {slices} slices)")
