"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the reference's own known-answer
vectors (tests/golden/kat.json) and (b) closed forms computed independently
with numpy -- IEEE binary16 casts, exact products, round-half-even ties --
chosen so that a plausible mistake (swapped nibbles, round-half-away, the
fp16 instead of the fp32 scale, a dropped subnormal) fails at least one of
them. The last tests plant such mistakes in copies of the oracle's logic and
show the checks reject them.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


def f16(a):
    return np.asarray(a, dtype=np.float16)


# ----------------------------------------------------------------- KATs ----
def test_kat_pack_unpack():
    assert oracle.pack_int4(KAT["pack_int4"]["codes"]).tolist() == KAT["pack_int4"]["packed"]
    assert oracle.unpack_int4(np.array(KAT["unpack_int4"]["packed"], np.uint8)).tolist() == KAT["unpack_int4"]["codes"]


def test_kat_quantize():
    k = KAT["quantize_groupwise"]
    q, s = oracle.quantize_groupwise(f16(k["weights_f16"]).astype(np.float32), k["group_size"])
    assert q.tolist() == k["codes"]
    assert s.tolist() == k["scales_f16"]
    k = KAT["quantize_and_pack"]
    p, s = oracle.quantize_and_pack(f16(k["weights_f16"]).astype(np.float32), k["group_size"])
    assert p.tolist() == k["packed"]
    assert s.tolist() == k["scales_f16"]


def test_kat_dequantize():
    k = KAT["dequantize"]
    p = oracle.pack_int4(k["codes"])
    w = oracle.dequantize_f32(p, f16(k["scales_f16"]), k["group_size"])
    assert w.dtype == np.float32 and w.tolist() == k["weights_f32"]


def test_kat_linear():
    k = KAT["linear"]
    p = oracle.pack_int4(k["codes"])
    out = oracle.linear(f16(k["activations_f16"]), p, f16(k["scales_f16"]), k["group_size"])
    assert out.dtype == np.float16 and out.tolist() == k["output_f16"]


# ------------------------------------------------------------ binary16 ----
def test_f16_to_f32_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits.view(np.float16))
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_trip_and_ties():
    # every finite binary16 value round-trips
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16)
    vals = vals[np.isfinite(vals)]
    assert np.array_equal(oracle.f32_to_f16(vals.astype(np.float32)).view(np.uint16), vals.view(np.uint16))
    # midpoints between consecutive positive binary16 values (normal and subnormal): ties to even
    pos = np.sort(vals[(vals > 0)].astype(np.float64))
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    exact = mids.astype(np.float64) == (pos[:-1] + pos[1:]) / 2   # midpoints representable in fp32
    got = oracle.f32_to_f16(mids[exact]).view(np.uint16)
    ref = mids[exact].astype(np.float16).view(np.uint16)         # numpy casts round to nearest even
    assert np.array_equal(got, ref)
    assert np.all(got % 2 == 0)                                   # a tie always lands on an even mantissa


def test_f32_to_f16_random_and_edges():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([65504.0, 65519.996, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                  2.0 ** -26, 6.1035156e-05, 6.1e-05, 0.0, -0.0, np.inf, -np.inf], dtype=np.float32),
    ])
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


# --------------------------------------------------------- pack/unpack ----
def test_unpack_all_bytes_closed_form():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    codes = oracle.unpack_int4(b)
    lo = ((b.astype(np.int16) & 15) ^ 8) - 8
    hi = ((b.astype(np.int16) >> 4) ^ 8) - 8
    assert np.array_equal(codes[:, 0::2], lo) and np.array_equal(codes[:, 1::2], hi)
    assert codes.min() == -8 and codes.max() == 7


def test_pack_is_inverse_of_unpack_on_quantizer_range():
    b = np.array([[x for x in range(256) if (x & 15) != 8 and (x >> 4) != 8]], dtype=np.uint8)
    assert np.array_equal(oracle.pack_int4(oracle.unpack_int4(b)), b)


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        oracle.pack_int4([[8, 0]])
    with pytest.raises(ValueError):
        oracle.pack_int4([[-8, 0]])


# ----------------------------------------------------------- quantizer ----
def test_quantize_round_half_even_ties():
    # amax 0.875 -> fp32 scale 0.125 exactly, so w/s lands exactly on .5 ties
    w = np.array([[0.875, 0.1875, 0.3125, -0.0625, 0.0625, -0.1875, 0.4375, 0.5625]], np.float32)
    q, s = oracle.quantize_groupwise(w, 8)
    assert q.tolist() == [[7, 2, 2, 0, 0, -2, 4, 4]]   # 1.5->2, 2.5->2, -0.5->0, 3.5->4, 4.5->4
    assert s.tolist() == [[0.125]]


def test_quantize_uses_fp32_scale_for_codes():
    # amax/7 is not a binary16 value, so w / fp32(s) and w / fp16(s) round differently for some w
    amax = np.float32(0.7)
    s32 = amax / np.float32(7.0)
    s16 = np.float32(np.float16(s32))
    # find a weight whose code differs between the two divisors
    cands = np.linspace(-0.7, 0.7, 20001, dtype=np.float32)
    diff = cands[np.rint(cands / s32) != np.rint(cands / s16)]
    assert diff.size > 0
    w = np.array([[amax, diff[0], 0.0, 0.0]], np.float32)
    q, s = oracle.quantize_groupwise(w, 4)
    assert q[0, 1] == np.rint(diff[0] / s32)
    assert s[0, 0] == np.float16(s32)


def test_quantize_invariants_random():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    w[3, 128:256] = 0.0                                      # an all-zero group
    q, s = oracle.quantize_groupwise(w, 128)
    g = w.reshape(64, 4, 128)
    qg = q.reshape(64, 4, 128)
    assert q.min() >= -7 and q.max() <= 7
    amax = np.abs(g).max(axis=2)
    # the group's absmax element maps to +-7 (scale = amax / 7 in fp32)
    idx = np.abs(g).argmax(axis=2)
    picked = np.take_along_axis(qg, idx[..., None], axis=2)[..., 0]
    nz = amax > 0
    assert np.array_equal(np.abs(picked[nz]), np.full(nz.sum(), 7))
    assert s[3, 1] == 1.0 and np.all(qg[3, 1] == 0)
    # stored scale: binary16 of the fp32 amax / 7 (numpy division and cast)
    ref = np.where(amax == 0, np.float32(1.0), amax.astype(np.float32) / np.float32(7.0)).astype(np.float16)
    assert np.array_equal(s.view(np.uint16), ref.view(np.uint16))
    # every code is the nearest integer to w/s32 (|w/s - q| <= 1/2)
    s32 = np.where(amax == 0, np.float32(1.0), amax.astype(np.float32) / np.float32(7.0))
    err = np.abs(g / s32[..., None] - qg)
    assert err.max() <= 0.5 + 1e-6


# ------------------------------------------------------------ dequant ----
def test_dequantize_f16_all_codes_all_scales_closed_form():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    scales = bits.view(np.float16).reshape(-1, 1)
    row = np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE] * 2, np.uint8)  # codes 0..7,-8..-1 twice
    packed = np.tile(row, (65536, 1))
    got = oracle.dequantize_f16(packed, scales, 32).astype(np.float64)
    codes = np.array(([0, 1, 2, 3, 4, 5, 6, 7, -8, -7, -6, -5, -4, -3, -2, -1]) * 2, np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = (codes[None, :] * scales.astype(np.float64)).astype(np.float16).astype(np.float64)  # one RNE
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    # signed zeros and subnormals kept bit for bit
    got_bits = oracle.dequantize_f16(packed, scales, 32).view(np.uint16)
    with np.errstate(invalid="ignore", over="ignore"):
        ref_bits = (codes[None, :] * scales.astype(np.float64)).astype(np.float16).view(np.uint16)
    assert np.array_equal(got_bits[~nan], ref_bits[~nan])


def test_dequantize_f32_exact_products():
    rng = np.random.default_rng(2)
    packed = rng.integers(0, 256, (16, 64), dtype=np.uint8)
    scales = (rng.random((16, 4)) * 3).astype(np.float16)
    w = oracle.dequantize_f32(packed, scales, 32)
    codes = oracle.unpack_int4(packed).astype(np.float64)
    ref = (codes.reshape(16, 4, 32) * scales.astype(np.float64)[..., None]).reshape(16, 128)
    assert np.array_equal(w.astype(np.float64), ref)


# ------------------------------------------------------------- linear ----
@pytest.mark.parametrize("m,k,n,g", [(1, 256, 8, 128), (3, 384, 19, 64), (8, 1024, 13, 128), (2, 96, 5, 6)])
def test_linear_matches_float64_brute_force(m, k, n, g):
    rng = np.random.default_rng(m * k + n)
    x = rng.standard_normal((m, k)).astype(np.float16)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = (rng.random((n, k // g)) + 0.01).astype(np.float16)
    out = oracle.linear(x, packed, scales, g).astype(np.float64)
    w = oracle.unpack_int4(packed).astype(np.float64).reshape(n, k // g, g) * scales.astype(np.float64)[..., None]
    ref = x.astype(np.float64) @ w.reshape(n, k).T
    # fp16 output: within half an ulp of the float64 value (plus the fp32 intermediate's rounding)
    assert np.all(np.abs(out - ref) <= np.abs(ref) * 2.0 ** -11 + 2.0 ** -24 + 1e-6 * np.abs(ref))


def test_linear_rejects_mismatched_k():
    with pytest.raises(ValueError):
        oracle.linear(np.zeros((1, 256), np.float16), np.zeros((8, 64), np.uint8), np.ones((8, 2), np.float16), 128)


# ---------------------------------------- planted mistakes must be caught ----
def _unpack_swapped(packed):
    b = np.asarray(packed, np.int16)
    out = np.empty((b.shape[0], 2 * b.shape[1]), np.int16)
    out[:, 0::2] = ((b >> 4) ^ 8) - 8     # mistake: high nibble first
    out[:, 1::2] = ((b & 15) ^ 8) - 8
    return out


def _quantize_half_away(w, g):
    wg = w.reshape(w.shape[0], -1, g)
    amax = np.abs(wg).max(axis=2, keepdims=True)
    s = np.where(amax == 0, np.float32(1), amax / np.float32(7))
    q = np.clip(np.sign(wg / s) * np.floor(np.abs(wg / s) + 0.5), -7, 7)   # mistake: round half away
    return q.reshape(w.shape).astype(np.int8)


def test_planted_nibble_swap_fails_kat():
    assert _unpack_swapped(np.array(KAT["unpack_int4"]["packed"])).tolist() != KAT["unpack_int4"]["codes"]


def test_planted_round_half_away_fails_tie_check():
    w = np.array([[0.875, 0.1875, 0.3125, -0.0625, 0.0625, -0.1875, 0.4375, 0.5625]], np.float32)
    assert _quantize_half_away(w, 8).tolist() != [[7, 2, 2, 0, 0, -2, 4, 4]]
