"""w4a16_linear_noalloc_f16 (the allocation-free entry point) through the C
ABI, against w4a16_linear_ws_f16 with a caller workspace (the same kernels:
bit-identical outputs) and the CPU oracle (|err| <= 1e-2 (1 + |ref|)), on
consecutive calls whose second is smaller, so partial sums the first call
left in the shared scratch cannot leak into the second; captured in a HIP
graph (its stated use) without any allocation; and a layer whose split-K
partials would pass the scratch, which takes the no-workspace route."""

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


def test_noalloc_graph_capture_allocates_nothing(gpu):
    """Warm-up call (the scratch address is looked up outside the capture),
    then the call captured with torch.cuda.graph and replayed three times with
    eager work between the replays: every replay equals the eager output bit
    for bit, and the caching allocator holds the same bytes throughout."""
    m, k, n = 8, 28672, 8192   # the split-K route: partial sums in the scratch
    x, p, s = make_case(m, k, n, seed=77)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    assert _lib.linear_workspace_bytes(m, n, k) > 0
    eager = torch.empty((m, n), dtype=torch.float16, device=gpu)
    out = torch.empty((m, n), dtype=torch.float16, device=gpu)
    print("[case] noalloc graph capture M=8 K=28672 N=8192", flush=True)
    _lib.linear_noalloc_f16(xd, pd, sd, eager)
    torch.cuda.synchronize()
    # a second split-K layer whose partial sums overwrite the scratch between replays
    x2, p2, s2 = make_case(3, 20480, 8200, seed=78, all_nibbles=True)
    assert _lib.linear_workspace_bytes(3, 8200, 20480) > 0
    small = (x2.to(gpu), p2.to(gpu), s2.to(gpu))
    other = torch.empty((3, 8200), dtype=torch.float16, device=gpu)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    # torch allocates its generator's graph state on the first capture of a
    # process: a capture of an in-place fill first, so the count below is the
    # call's alone
    warm = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(warm, stream=stream):
            other.zero_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    before = torch.cuda.memory_allocated(gpu)
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _lib.linear_noalloc_f16(xd, pd, sd, out)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(gpu) == before
    for r in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {r}"
        _lib.linear_noalloc_f16(*small, other)   # eager work on the same scratch between replays
        torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(gpu) == before
    assert_parity(out, expected(x, p, s), "noalloc graph replay")


def test_noalloc_partials_past_scratch_take_unsplit_route(gpu):
    """M = 8, K = 20480, N = 66000: four K slices of fp32 partials would need
    8.4 MB, past the 8 MiB scratch, so the call takes w4a16_linear_f16's route
    (no workspace): bit-identical to it, and to the oracle on sampled rows."""
    m, k, n = 8, 20480, 66000
    need = _lib.linear_workspace_bytes(m, n, k)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    gen = torch.Generator(device=gpu).manual_seed(5)
    pd = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=gpu, generator=gen)
    sd = (torch.rand((n, k // 128), device=gpu, generator=gen) * 0.01 + 0.001).to(torch.float16)
    xd = torch.randn((m, k), device=gpu, generator=gen).to(torch.float16)
    out = torch.full((m, n), float("nan"), dtype=torch.float16, device=gpu)
    ref = torch.full((m, n), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] noalloc past scratch M={m} K={k} N={n} need={need}", flush=True)
    _lib.linear_noalloc_f16(xd, pd, sd, out)
    _lib.linear_f16(xd, pd, sd, ref, workspace=None)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    rows = torch.cat([torch.arange(0, 96), torch.arange(n - 96, n)]).to(gpu)
    assert_parity(out[:, rows], expected(xd.cpu(), pd[rows].cpu(), sd[rows].cpu()), "noalloc past scratch")
