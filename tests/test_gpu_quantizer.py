"""The quantizer run on GPU tensors (``quantize_and_pack_weights`` on cuda,
as the bench, the decoder and the full-size GPU tests call it) against the
CPU oracle's restatement of reference ``w4a16/quantization.py:65-113``:
packed bytes and fp16 scale bits must be identical. Every GPU parity test
takes its weights from this path, so a device-side difference in the fp32
division, the round-half-even or the fp16 cast would otherwise go unseen."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

import oracle
from nibble_amd.quantization import quantize_and_pack_weights, quantize_groupwise

pytestmark = pytest.mark.gpu

KAT = os.path.join(os.path.dirname(__file__), "golden", "kat.json")


def _device_quantize(w: np.ndarray, group: int, dev):
    p, s = quantize_and_pack_weights(torch.from_numpy(w).to(dev), group)
    torch.cuda.synchronize()
    return p.cpu().numpy(), s.cpu().numpy()


def _assert_same(w: np.ndarray, group: int, dev, what: str):
    print(f"[case] {what} shape={w.shape} G={group}", flush=True)
    p, s = _device_quantize(w, group, dev)
    rp, rs = oracle.quantize_and_pack(w, group)
    assert p.dtype == np.uint8 and s.dtype == np.float16
    bad = np.argwhere(p != rp)
    assert bad.size == 0, f"{what}: {len(bad)} packed bytes differ, first at {bad[:3].tolist()}"
    assert np.array_equal(s.view(np.uint16), rs.view(np.uint16)), f"{what}: fp16 scale bits differ"


@pytest.mark.parametrize("k,n", [(2048, 5632), (5632, 2048), (4096, 14336)])
def test_device_quantizer_configs_shapes(gpu, k, n):
    """The configs shapes from N(0, 0.02) fp32 weights, as the benchmark makes
    them ([N, K], group 128)."""
    rng = np.random.default_rng(k + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    _assert_same(w, 128, gpu, f"N(0,0.02) {n}x{k}")


def test_device_quantizer_kats(gpu):
    """The reference's known answers (tests/test_quantization.py:51-90)."""
    with open(KAT) as f:
        kat = json.load(f)
    q = kat["quantize_groupwise"]
    w = np.array(q["weights_f16"], dtype=np.float16)
    codes, scales = quantize_groupwise(torch.from_numpy(w).to(gpu), q["group_size"])
    torch.cuda.synchronize()
    assert codes.cpu().tolist() == q["codes"]
    assert scales.cpu().float().tolist() == q["scales_f16"]
    qp = kat["quantize_and_pack"]
    w = np.array(qp["weights_f16"], dtype=np.float16)
    packed, scales = quantize_and_pack_weights(torch.from_numpy(w).to(gpu), qp["group_size"])
    torch.cuda.synchronize()
    assert packed.cpu().tolist() == qp["packed"]
    assert scales.cpu().float().tolist() == qp["scales_f16"]


def test_device_quantizer_ties(gpu):
    """Groups of amax 0.875 (fp32 scale exactly 0.125) whose other weights sit
    on every half-integer multiple of the scale, so w / s lands exactly on .5
    ties and the round must go to even, as on the CPU."""
    halves = (np.arange(-13, 14, dtype=np.float32) * 0.0625)    # k * s / 2 for s = 0.125
    g = 128
    rows = []
    for r in range(64):
        row = np.resize(np.roll(halves, r), g).astype(np.float32)
        row[r % g] = 0.875 if r % 2 == 0 else -0.875
        rows.append(row)
    w = np.concatenate([np.stack(rows), np.zeros((64, g), np.float32)], axis=1)   # a zero group too (scale 1.0)
    _assert_same(w, g, gpu, "ties")
    codes, _ = oracle.quantize_groupwise(w, g)
    assert np.all(np.abs(codes[:, :g]) <= 7) and np.all(codes[:, g:] == 0)


def test_device_quantizer_wide_range_and_fp16_input(gpu):
    """Magnitudes over many decades (subnormal fp16 scales included) and fp16
    weights, group sizes 32 and 128."""
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((96, 1024)) * np.exp(rng.uniform(-18, 4, (96, 1)))).astype(np.float32)
    _assert_same(w, 128, gpu, "wide range fp32")
    _assert_same(w, 32, gpu, "wide range fp32 G=32")
    w16 = (rng.standard_normal((64, 512)) * 0.05).astype(np.float16)
    p, s = _device_quantize(w16, 128, gpu)
    rp, rs = oracle.quantize_and_pack(w16.astype(np.float32), 128)
    assert np.array_equal(p, rp) and np.array_equal(s.view(np.uint16), rs.view(np.uint16))
