"""Shared input generators and the parity check used by the GPU tests."""

from __future__ import annotations

import numpy as np
import torch

import oracle
from nibble_amd.quantization import quantize_and_pack_weights


def make_case(m: int, k: int, n: int, seed: int = 0, all_nibbles: bool = False, group_size: int = 128,
              device: str = "cpu"):
    """FP16 activations ~N(0,1); INT4 weights quantized from ~N(0,0.02) fp32
    (or uniformly random bytes with scales in [0.01, 1.01) when all_nibbles,
    which reaches code -8 the quantizer never emits). CPU tensors."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=gen).to(torch.float16)
    if all_nibbles:
        packed = torch.randint(0, 256, (n, k // 2), generator=gen, dtype=torch.uint8)
        scales = (torch.rand((n, k // group_size), generator=gen) + 0.01).to(torch.float16)
    else:
        w = torch.randn((n, k), generator=gen) * 0.02
        if device != "cpu":
            packed, scales = quantize_and_pack_weights(w.to(device), group_size)
            packed, scales = packed.cpu(), scales.cpu()
        else:
            packed, scales = quantize_and_pack_weights(w, group_size)
    return x, packed, scales


def expected(x, packed, scales, group_size: int = 128) -> np.ndarray:
    return oracle.linear(x.numpy(), packed.numpy(), scales.numpy(), group_size).astype(np.float32)


def assert_parity(out: torch.Tensor, ref: np.ndarray, what: str = "") -> None:
    """|err| <= 1e-2 * (1 + |ref|) elementwise (the reference's rtol=atol=1e-2)."""
    got = out.detach().cpu().float().numpy()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = 1e-2 * (1.0 + np.abs(ref))
    bad = err > bound
    if bad.any():
        idx = np.argwhere(bad)[:5].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; max err {err.max():.4e}; "
                             f"first bad {idx}")
