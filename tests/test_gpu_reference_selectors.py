"""The reference's selector tests (tests/test_cuda.py:203-313) on this build:
W4A16_DECODE = v1..v4 and W4A16_ROWS_PER_WARP through torch.ops.w4a16.linear,
with the reference's inputs (fp16 randn weights quantized on the device,
uniformly random bytes for the all-nibble case), checked against the CPU
oracle on the same packed bytes at the reference's bar |err| <= 1e-2 (1 + |ref|).
"""

from __future__ import annotations

import pytest
import torch

from nibble_amd import _lib
from w4a16.cuda import linear_cuda
from w4a16.quantization import quantize_and_pack_weights
from tests._cases import assert_parity, expected

pytestmark = pytest.mark.gpu


def _quantized(k: int, n: int, m: int, dev):
    torch.manual_seed(0)
    x = torch.randn((m, k), dtype=torch.float16, device=dev)
    w = torch.randn((n, k), dtype=torch.float16, device=dev)
    packed, scales = quantize_and_pack_weights(w, group_size=128)
    return x, packed, scales


def _check(out, x, packed, scales, what: str, kernel: str | None = None) -> None:
    torch.cuda.synchronize()
    if kernel is not None:
        plan = _lib.plan_linear(x.data_ptr(), packed.data_ptr(), x.shape[0], packed.shape[0], x.shape[1])
        assert plan["kernel"] == kernel, (what, plan)
    assert_parity(out, expected(x.cpu(), packed.cpu(), scales.cpu()), what)


VERSION_KERNEL = {"v1": "valu", "v2": "diag", "v3": "valu_offset", "v4": "oneshot"}


@pytest.mark.parametrize("version", ["v1", "v2", "v3", "v4"])
def test_decode_versions_match_oracle(gpu, monkeypatch, version):
    """Reference tests/test_cuda.py:203-225: each version at M = 1, 2048 x 2048."""
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    x, packed, scales = _quantized(2048, 2048, 1, gpu)
    monkeypatch.setenv("W4A16_DECODE", version)
    print(f"[case] W4A16_DECODE={version} M=1 K=2048 N=2048", flush=True)
    out = linear_cuda(x, packed, scales, group_size=128)
    _check(out, x, packed, scales, f"{version} 2048x2048", VERSION_KERNEL[version])


@pytest.mark.parametrize("version", ["v1", "v2", "v3", "v4"])
def test_decode_versions_all_nibbles(gpu, monkeypatch, version):
    """Reference tests/test_cuda.py:228-256: random bytes reach every code,
    -8 included, in both nibbles of every byte position."""
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    torch.manual_seed(0)
    x = torch.randn((1, 1024), dtype=torch.float16, device=gpu)
    packed = torch.randint(0, 256, (64, 512), dtype=torch.uint8, device=gpu)
    scales = torch.rand((64, 8), device=gpu).add(0.01).to(torch.float16)
    monkeypatch.setenv("W4A16_DECODE", version)
    print(f"[case] W4A16_DECODE={version} all nibbles M=1 K=1024 N=64", flush=True)
    out = linear_cuda(x, packed, scales, group_size=128)
    _check(out, x, packed, scales, f"{version} all nibbles", VERSION_KERNEL[version])


@pytest.mark.parametrize("rows_per_warp", ["1", "2", "4"])
@pytest.mark.parametrize("k,n", [(256, 7), (1024, 13), (2048, 2048), (5632, 2048), (2048, 5632)])
def test_v4_rows_per_warp(gpu, monkeypatch, rows_per_warp, k, n):
    """Reference tests/test_cuda.py:259-295: v4 with 1, 2 and 4 rows per
    wavefront; N = 7 and 13 leave a partial last wavefront."""
    x, packed, scales = _quantized(k, n, 1, gpu)
    monkeypatch.setenv("W4A16_DECODE", "v4")
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", rows_per_warp)
    print(f"[case] v4 rows={rows_per_warp} M=1 K={k} N={n}", flush=True)
    out = linear_cuda(x, packed, scales, group_size=128)
    torch.cuda.synchronize()
    plan = _lib.plan_linear(x.data_ptr(), packed.data_ptr(), 1, n, k)
    assert (plan["kernel"], plan["rows"]) == ("valu", int(rows_per_warp))
    _check(out, x, packed, scales, f"v4 rows={rows_per_warp} K={k} N={n}")


def test_v4_rejects_bad_rows_per_warp(gpu, monkeypatch):
    """Reference tests/test_cuda.py:298-313."""
    x, packed, scales = _quantized(256, 8, 1, gpu)
    monkeypatch.setenv("W4A16_DECODE", "v4")
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "3")
    with pytest.raises(RuntimeError, match="W4A16_ROWS_PER_WARP must be 1, 2, or 4"):
        linear_cuda(x, packed, scales, group_size=128)


@pytest.mark.parametrize("m", [2, 4, 8])
def test_rows_per_warp_ignored_off_the_m1_path(gpu, monkeypatch, m):
    """The reference reads W4A16_ROWS_PER_WARP only at M = 1 (:713-749), so a
    bad value leaves small batches, and v1 at M = 1, running."""
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "3")
    monkeypatch.setenv("W4A16_DECODE", "v4")
    x, packed, scales = _quantized(2048, 512, m, gpu)
    print(f"[case] rows=3 M={m} K=2048 N=512", flush=True)
    out = linear_cuda(x, packed, scales, group_size=128)
    _check(out, x, packed, scales, f"rows=3 M={m}")
    if m == 2:
        monkeypatch.setenv("W4A16_DECODE", "v1")
        x1 = x[:1].contiguous()
        out = linear_cuda(x1, packed, scales, group_size=128)
        _check(out, x1, packed, scales, "v1 with rows=3", "valu")


@pytest.mark.parametrize("version", ["v2", "nonsense", ""])
def test_unknown_and_m1_only_versions_at_small_batch(gpu, monkeypatch, version):
    """v1..v3 select M = 1 kernels only; unknown values are the default."""
    monkeypatch.delenv("W4A16_ROWS_PER_WARP", raising=False)
    monkeypatch.setenv("W4A16_DECODE", version)
    for m in (1, 4):
        x, packed, scales = _quantized(5632, 2048, m, gpu)
        print(f"[case] W4A16_DECODE={version!r} M={m} K=5632 N=2048", flush=True)
        out = linear_cuda(x, packed, scales, group_size=128)
        _check(out, x, packed, scales, f"{version!r} M={m}")
