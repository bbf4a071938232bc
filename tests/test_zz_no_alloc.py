"""w4a16_linear_noalloc_f16 (the allocation-free entry point) through the C
ABI, against w4a16_linear_ws_f16 with a caller workspace (the same kernels:
bit-identical outputs) and the CPU oracle (|err| <= 1e-2 (1 + |ref|)), on
consecutive calls whose second is smaller, so partial sums the first call
left in the shared scratch cannot leak into the second."""

from __future__ import annotations

import pytest
import torch

from nibble_amd import _lib
from tests._cases import assert_parity, expected, make_case

pytestmark = pytest.mark.gpu


def _both(dev, m, k, n, seed):
    x, p, s = make_case(m, k, n, seed=seed)
    xd, pd, sd = x.to(dev), p.to(dev), s.to(dev)
    ref_out = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    out = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    nbytes = _lib.linear_workspace_bytes(m, n, k)
    ws = torch.full((max(1, nbytes // 4),), float("nan"), dtype=torch.float32, device=dev)
    print(f"[case] noalloc M={m} K={k} N={n} scratch={nbytes} B", flush=True)
    _lib.linear_f16(xd, pd, sd, ref_out, workspace=ws if nbytes > 0 else None)
    _lib.linear_noalloc_f16(xd, pd, sd, out)
    torch.cuda.synchronize()
    return x, p, s, out, ref_out, nbytes


@pytest.mark.parametrize("calls", [
    [(8, 28672, 8192), (3, 20480, 8200)],     # split-K twice, the second layer smaller
    [(6, 20480, 8200), (2, 2048, 5632), (4, 16512, 8192)],   # split-K, no scratch, split-K
])
def test_noalloc_matches_workspace_entry_point(gpu, calls):
    for i, (m, k, n) in enumerate(calls):
        x, p, s, out, ref_out, nbytes = _both(gpu, m, k, n, seed=31 * i + m + k)
        assert 0 < nbytes <= _lib.NOALLOC_SCRATCH_BYTES or m < 3
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), (m, k, n)
        assert_parity(out, expected(x, p, s), f"noalloc M={m} K={k} N={n}")


def test_noalloc_small_layers_and_empty(gpu):
    for m, k, n in [(1, 4096, 14336), (8, 5632, 2048), (16, 2048, 2048)]:
        x, p, s, out, ref_out, nbytes = _both(gpu, m, k, n, seed=m)
        assert nbytes == 0
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), (m, k, n)
        assert_parity(out, expected(x, p, s), f"noalloc M={m} K={k} N={n}")
    empty = torch.empty((0, 256), dtype=torch.float16, device=gpu)
    p = torch.zeros((8, 128), dtype=torch.uint8, device=gpu)
    s = torch.ones((8, 2), dtype=torch.float16, device=gpu)
    _lib.linear_noalloc_f16(empty, p, s, torch.empty((0, 8), dtype=torch.float16, device=gpu))
