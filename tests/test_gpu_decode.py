"""GPU tests of the decode-step entry points (include/w4a16_decode.h), called
through the C ABI, and of the Llama decoder's fused step.

References: the fused GEMV against the CPU oracle applied to the torch-fp32
RMSNorm of the row (bar |err| <= 1e-2 (1 + |ref|), with the residual add and
SiLU-multiply done on fp16-rounded values as fp16 tensors would); attention
against a float64 torch restatement of rotary embedding + masked softmax
attention (|err| <= 2e-3 + 1e-2 |ref|, fp16 output); argmax and embedding
exactly."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from nibble_amd import _lib
from tests._cases import assert_parity, make_case

pytestmark = pytest.mark.gpu


def _rms_norm_f16(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * w.float()).to(torch.float16)


def _linear_ref(x16: torch.Tensor, p: torch.Tensor, s: torch.Tensor) -> np.ndarray:
    return oracle.linear(x16.cpu().numpy().reshape(1, -1), p.cpu().numpy(), s.cpu().numpy(), 128)[0]


def _f16(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("k,n", [(256, 7), (2048, 64), (2048, 2560), (5632, 300), (16384, 33), (2048, 32000),
                                 (2048, 20004)])
@pytest.mark.parametrize("norm", [False, True])
def test_gemv_fused_plain_and_norm(gpu, k, n, norm):
    """One row (the decode step's q|k|v and lm_head): the one-shot kernel, or
    with RMSNorm on rows of 2048 of wide layers the ring kernel's RMSNorm
    prologue; against the oracle on the fp16 RMSNorm of the row."""
    x, p, s = make_case(1, k, n, seed=k + n)
    gen = torch.Generator().manual_seed(k)
    w = (1.0 + 0.5 * torch.randn((k,), generator=gen)).to(torch.float16)
    xin = _rms_norm_f16(x, w, 1e-5) if norm else x
    ref = _linear_ref(xin, p, s)
    out = torch.full((n,), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] fused norm={norm} K={k} N={n}", flush=True)
    _lib.gemv_fused_f16(x.to(gpu), p.to(gpu), s.to(gpu), out, norm_weight=w.to(gpu) if norm else None, eps=1e-5)
    torch.cuda.synchronize()
    assert_parity(out.view(1, n), ref.reshape(1, n), f"fused norm={norm} K={k} N={n}")


@pytest.mark.parametrize("alias", [False, True])
@pytest.mark.parametrize("k,n", [(2048, 2048), (5632, 2048), (256, 9), (5632, 2003)])
def test_gemv_fused_residual(gpu, k, n, alias):
    """The residual add (in place or not): rows of 5632 on the ring kernel's
    residual epilogue (ragged N too), others on the one-shot kernel."""
    x, p, s = make_case(1, k, n, seed=3 * k + n)
    resid = torch.randn((n,), generator=torch.Generator().manual_seed(n)).to(torch.float16)
    ref = _f16(resid.float().numpy() + _f16(_linear_ref(x, p, s)))
    r = resid.to(gpu)
    out = r if alias else torch.full((n,), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] fused residual alias={alias} K={k} N={n}", flush=True)
    _lib.gemv_fused_f16(x.to(gpu), p.to(gpu), s.to(gpu), out, residual=r)
    torch.cuda.synchronize()
    assert_parity(out.view(1, n), ref.reshape(1, n), f"residual alias={alias}")


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("k,half", [(2048, 5632), (256, 5), (4096, 64), (2048, 5000), (2048, 24)])
def test_gemv_fused_paired_silu(gpu, k, half, norm):
    """gate|up with SiLU * up: rows of 2048 on the ring kernel's SiLU form
    (a gate and an up block per wavefront; ragged and tiny layers), others on
    the one-shot kernel's paired rows."""
    x, p, s = make_case(1, k, 2 * half, seed=k + half)
    w = (1.0 + 0.25 * torch.randn((k,), generator=torch.Generator().manual_seed(7))).to(torch.float16)
    xin = _rms_norm_f16(x, w, 1e-6) if norm else x
    y = _f16(_linear_ref(xin, p, s))
    g, u = y[:half].astype(np.float64), y[half:].astype(np.float64)
    ref = _f16(_f16(g / (1.0 + np.exp(-g))) * u)
    out = torch.full((half,), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] fused paired norm={norm} K={k} N/2={half}", flush=True)
    _lib.gemv_fused_f16(x.to(gpu), p.to(gpu), s.to(gpu), out, norm_weight=w.to(gpu) if norm else None, eps=1e-6,
                        paired=True)
    torch.cuda.synchronize()
    assert_parity(out.view(1, half), ref.reshape(1, half), f"paired norm={norm}")


def test_gemv_fused_rejects(gpu):
    x, p, s = make_case(1, 256, 7, seed=1)
    out = torch.empty((7,), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="even number of rows"):
        _lib.gemv_fused_f16(x.to(gpu), p.to(gpu), s.to(gpu), out, paired=True)
    xd = torch.empty((257,), dtype=torch.float16, device=gpu)[1:]
    with pytest.raises(_lib.W4A16Error, match="16-byte aligned"):
        _lib.gemv_fused_f16(xd, p.to(gpu), s.to(gpu), out)


# ------------------------------------------------------------ attention ----
def _rope64(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    x1, x2 = x[..., :32].double(), x[..., 32:].double()
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


def _tables(S: int, theta: float = 10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, 64, 2).float() / 64))
    ang = torch.outer(torch.arange(S).float(), inv)
    return ang.cos(), ang.sin()


@pytest.mark.parametrize("heads,kv", [(32, 4), (8, 8), (4, 1)])
@pytest.mark.parametrize("pos", [0, 1, 17, 63, 64, 127, 200, 511])
def test_decode_attention(gpu, heads, kv, pos):
    S = 512
    gen = torch.Generator().manual_seed(pos * 31 + heads)
    qkv = torch.randn(((heads + 2 * kv) * 64,), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    cos, sin = _tables(S)
    # reference (float64 on fp16-rounded rotary outputs, as the cache stores them)
    c, s_ = cos[pos].double(), sin[pos].double()
    q = _rope64(qkv[: heads * 64].view(heads, 64), c, s_).to(torch.float16).double()
    k_new = _rope64(qkv[heads * 64: (heads + kv) * 64].view(kv, 64), c, s_).to(torch.float16)
    v_new = qkv[(heads + kv) * 64:].view(kv, 64)
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, pos], vc[:, pos] = k_new, v_new
    group = heads // kv
    kf = kc.double().repeat_interleave(group, 0)[:, : pos + 1]
    vf = vc.double().repeat_interleave(group, 0)[:, : pos + 1]
    scores = torch.einsum("hd,hsd->hs", q, kf) / math.sqrt(64)
    ref = torch.einsum("hs,hsd->hd", torch.softmax(scores, dim=-1), vf).reshape(-1)

    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    out = torch.full((heads * 64,), float("nan"), dtype=torch.float16, device=gpu)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    print(f"[case] attention heads={heads} kv={kv} pos={pos}", flush=True)
    _lib.decode_attention_f16(qkv.to(gpu), kd, vd, cos.to(gpu), sin.to(gpu), position, out, heads, kv)
    torch.cuda.synchronize()
    got = out.double().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert float(err.max()) <= float((2e-3 + 1e-2 * ref.abs()).max()), float(err.max())
    assert torch.all(err <= 2e-3 + 1e-2 * ref.abs())
    # the cache gained exactly slot `pos` (rotary k within one fp16 ulp, v exact); other slots untouched
    kg, vg = kd.cpu(), vd.cpu()
    others = [t for t in range(S) if t != pos]
    assert torch.equal(kg[:, others], k_cache[:, others]) and torch.equal(vg[:, others], v_cache[:, others])
    assert torch.equal(vg[:, pos], v_new)
    assert torch.allclose(kg[:, pos].float(), k_new.float(), rtol=2 ** -10, atol=2 ** -14)


def _decode_case(heads, kv, pos, S, seed):
    """Inputs and the float64 reference of one decode-attention call (as
    test_decode_attention builds them)."""
    gen = torch.Generator().manual_seed(seed)
    qkv = torch.randn(((heads + 2 * kv) * 64,), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    cos, sin = _tables(S)
    c, s_ = cos[pos].double(), sin[pos].double()
    q = _rope64(qkv[: heads * 64].view(heads, 64), c, s_).to(torch.float16).double()
    k_new = _rope64(qkv[heads * 64: (heads + kv) * 64].view(kv, 64), c, s_).to(torch.float16)
    v_new = qkv[(heads + kv) * 64:].view(kv, 64)
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, pos], vc[:, pos] = k_new, v_new
    group = heads // kv
    kf = kc.double().repeat_interleave(group, 0)[:, : pos + 1]
    vf = vc.double().repeat_interleave(group, 0)[:, : pos + 1]
    scores = torch.einsum("hd,hsd->hs", q, kf) / math.sqrt(64)
    ref = torch.einsum("hs,hsd->hd", torch.softmax(scores, dim=-1), vf).reshape(-1)
    return qkv, k_cache, v_cache, cos, sin, ref, k_new, v_new


@pytest.mark.parametrize("splits", [1, 3, 8, 64])
@pytest.mark.parametrize("heads,kv", [(32, 4), (8, 8), (4, 1)])
@pytest.mark.parametrize("pos", [0, 63, 64, 200, 511, 1500, 2047])
def test_decode_attention_split(gpu, heads, kv, pos, splits):
    """The split form (a workgroup per head and share of the slots, merged per
    head) against the float64 reference, within the unsplit form's bound;
    shares past the position (no slots) included; the new k / v rows
    appended once, every other slot untouched."""
    S = 2048
    qkv, k_cache, v_cache, cos, sin, ref, k_new, v_new = _decode_case(heads, kv, pos, S, pos * 7 + heads + splits)
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    out = torch.full((heads * 64,), float("nan"), dtype=torch.float16, device=gpu)
    ws = torch.full((heads * splits * 66,), float("nan"), dtype=torch.float32, device=gpu)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    print(f"[case] split attention heads={heads} kv={kv} pos={pos} splits={splits}", flush=True)
    _lib.decode_attention_split_f16(qkv.to(gpu), kd, vd, cos.to(gpu), sin.to(gpu), position, out, heads, kv,
                                    splits, ws)
    torch.cuda.synchronize()
    got = out.double().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert torch.all(err <= 2e-3 + 1e-2 * ref.abs()), float(err.max())
    kg, vg = kd.cpu(), vd.cpu()
    others = [t for t in range(S) if t != pos]
    assert torch.equal(kg[:, others], k_cache[:, others]) and torch.equal(vg[:, others], v_cache[:, others])
    assert torch.equal(vg[:, pos], v_new)
    assert torch.allclose(kg[:, pos].float(), k_new.float(), rtol=2 ** -10, atol=2 ** -14)


def test_decode_attention_split_out_of_range_and_rejects(gpu):
    S, heads, kv = 256, 8, 2
    qkv = torch.randn(((heads + 2 * kv) * 64,)).to(torch.float16).to(gpu)
    kd = torch.zeros((kv, S, 64), dtype=torch.float16, device=gpu)
    vd = torch.zeros_like(kd)
    cos, sin = _tables(S)
    cos, sin = cos.to(gpu), sin.to(gpu)
    out = torch.zeros((heads * 64,), dtype=torch.float16, device=gpu)
    ws = torch.zeros((heads * 4 * 66,), dtype=torch.float32, device=gpu)
    for bad in (S, -1):
        position = torch.tensor([bad], dtype=torch.int64, device=gpu)
        _lib.decode_attention_split_f16(qkv, kd, vd, cos, sin, position, out, heads, kv, 4, ws)
        torch.cuda.synchronize()
        assert torch.isnan(out).all()
        assert not kd.any() and not vd.any()
    position = torch.tensor([3], dtype=torch.int64, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="workspace"):
        _lib.decode_attention_split_f16(qkv, kd, vd, cos, sin, position, out, heads, kv, 5, ws)
    for bad_splits in (0, 65):
        with pytest.raises(_lib.W4A16Error, match="splits"):
            _lib.decode_attention_split_f16(qkv, kd, vd, cos, sin, position, out, heads, kv, bad_splits, ws)
    assert not kd.any() and not vd.any()


def test_decode_attention_position_out_of_range(gpu):
    S, heads, kv = 16, 8, 2
    qkv = torch.randn(((heads + 2 * kv) * 64,)).to(torch.float16).to(gpu)
    kd = torch.zeros((kv, S, 64), dtype=torch.float16, device=gpu)
    vd = torch.zeros_like(kd)
    cos, sin = _tables(S)
    out = torch.zeros((heads * 64,), dtype=torch.float16, device=gpu)
    for bad in (S, -1):
        position = torch.tensor([bad], dtype=torch.int64, device=gpu)
        _lib.decode_attention_f16(qkv, kd, vd, cos.to(gpu), sin.to(gpu), position, out, heads, kv)
        torch.cuda.synchronize()
        assert torch.isnan(out).all()
        assert not kd.any() and not vd.any()


# ------------------------------------------------ attention + o projection ----
def _inv_freq(theta: float = 10000.0) -> torch.Tensor:
    return 1.0 / (theta ** (torch.arange(0, 64, 2).float() / 64))


def _attention_ref(qkv, k_cache, v_cache, pos, heads, kv):
    """float64 attention of the new token with cos / sin of the fp32 angle
    pos * inv_freq (as the kernel forms it); returns (attn [heads*64] float64,
    rotated k_new fp16, v_new fp16)."""
    ang = (torch.tensor(float(pos)) * _inv_freq()).double()
    c, s_ = ang.cos(), ang.sin()
    q = _rope64(qkv[: heads * 64].view(heads, 64), c, s_).to(torch.float16).double()
    k_new = _rope64(qkv[heads * 64: (heads + kv) * 64].view(kv, 64), c, s_).to(torch.float16)
    v_new = qkv[(heads + kv) * 64:].view(kv, 64)
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, pos], vc[:, pos] = k_new, v_new
    group = heads // kv
    kf = kc.double().repeat_interleave(group, 0)[:, : pos + 1]
    vf = vc.double().repeat_interleave(group, 0)[:, : pos + 1]
    scores = torch.einsum("hd,hsd->hs", q, kf) / math.sqrt(64)
    attn = torch.einsum("hs,hsd->hd", torch.softmax(scores, dim=-1), vf).reshape(-1)
    return attn, k_new, v_new


_DIAG = 7 * float(torch.tensor(1.0 / 7.0, dtype=torch.float16))   # code 7 x fp16(1/7)


def _identity_o(n: int):
    """INT4 packing of _DIAG times the n x n identity (code 7, every scale
    fp16(1/7): the magnitudes of a real layer, where the offset decode's fp32
    rounding is ~1e-3 of a chunk's activations times the scale)."""
    codes = torch.zeros((n, n), dtype=torch.int8)
    codes[torch.arange(n), torch.arange(n)] = 7
    lo, hi = codes[:, 0::2].to(torch.uint8) & 0xF, codes[:, 1::2].to(torch.uint8) & 0xF
    return lo | (hi << 4), torch.full((n, n // 128), 1.0 / 7.0, dtype=torch.float16)


@pytest.mark.parametrize("heads,kv", [(32, 4), (8, 2), (4, 1), (64, 8), (16, 1)])
@pytest.mark.parametrize("pos,S", [(0, 48), (1, 48), (17, 48), (47, 48), (63, 64), (40, 512), (63, 512)])
def test_attention_o_identity_projection(gpu, heads, kv, pos, S):
    """With o = _DIAG x identity and a zero residual the output is the
    attention row itself times _DIAG (rounded to fp16): the bar of the
    attention test, |err| <= 2e-3 + 1e-2 |ref|; slots past the position hold
    NaN, which must not leak in; the cache gains exactly slot pos."""
    gen = torch.Generator().manual_seed(pos * 131 + heads + S)
    qkv = torch.randn(((heads + 2 * kv) * 64,), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    k_cache[:, pos + 1:] = float("nan")
    v_cache[:, pos + 1:] = float("nan")
    ref, k_new, v_new = _attention_ref(qkv, k_cache, v_cache, pos, heads, kv)
    ref = ref * _DIAG
    n = heads * 64
    op, os_ = _identity_o(n)
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    resid = torch.zeros((n,), dtype=torch.float16, device=gpu)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    print(f"[case] attention_o identity heads={heads} kv={kv} pos={pos} S={S}", flush=True)
    _lib.attention_o_f16(qkv.to(gpu), kd, vd, _inv_freq().to(gpu), position, op.to(gpu), os_.to(gpu), resid,
                         heads, kv)
    torch.cuda.synchronize()
    got = resid.double().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert torch.all(err <= 2e-3 + 1e-2 * ref.abs()), float(err.max())
    kg, vg = kd.cpu(), vd.cpu()
    others = [t for t in range(S) if t != pos]
    assert torch.equal(kg[:, others].isnan(), k_cache[:, others].isnan())
    fin = [t for t in others if t < pos]
    assert torch.equal(kg[:, fin], k_cache[:, fin]) and torch.equal(vg[:, fin], v_cache[:, fin])
    assert torch.equal(vg[:, pos], v_new)
    assert torch.allclose(kg[:, pos].float(), k_new.float(), rtol=2 ** -10, atol=2 ** -14)


@pytest.mark.parametrize("heads,kv,hidden", [(32, 4, 2048), (8, 2, 300), (64, 8, 1000)])
@pytest.mark.parametrize("pos", [5, 47])
def test_attention_o_projection_and_residual(gpu, heads, kv, hidden, pos):
    """Random INT4 o projection (CPU oracle on the fp16-rounded attention row)
    plus a residual: out = fp16(resid + fp16(o . attn)), |err| <= 1e-2 (1 + |ref|)."""
    S = 48
    gen = torch.Generator().manual_seed(pos + hidden)
    qkv = torch.randn(((heads + 2 * kv) * 64,), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    attn, _, _ = _attention_ref(qkv, k_cache, v_cache, pos, heads, kv)
    _, op, os_ = make_case(1, heads * 64, hidden, seed=hidden)
    resid = torch.randn((hidden,), generator=gen).to(torch.float16)
    ref = _f16(resid.float().numpy() + _f16(_linear_ref(attn.to(torch.float16), op, os_)))
    out = resid.to(gpu)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    print(f"[case] attention_o projection heads={heads} kv={kv} hidden={hidden} pos={pos}", flush=True)
    _lib.attention_o_f16(qkv.to(gpu), k_cache.to(gpu), v_cache.to(gpu), _inv_freq().to(gpu), position, op.to(gpu),
                         os_.to(gpu), out, heads, kv)
    torch.cuda.synchronize()
    assert_parity(out.view(1, hidden), ref.reshape(1, hidden), f"attention_o heads={heads} hidden={hidden}")


def test_attention_o_position_out_of_range(gpu):
    heads, kv = 8, 2
    qkv = torch.randn(((heads + 2 * kv) * 64,)).to(torch.float16).to(gpu)
    op, os_ = _identity_o(heads * 64)
    op, os_ = op.to(gpu), os_.to(gpu)
    for S, bad in ((48, 48), (48, -1), (128, 64), (128, 100)):
        kd = torch.zeros((kv, S, 64), dtype=torch.float16, device=gpu)
        vd = torch.zeros_like(kd)
        resid = torch.zeros((heads * 64,), dtype=torch.float16, device=gpu)
        position = torch.tensor([bad], dtype=torch.int64, device=gpu)
        print(f"[case] attention_o out of range S={S} pos={bad}", flush=True)
        _lib.attention_o_f16(qkv, kd, vd, _inv_freq().to(gpu), position, op, os_, resid, heads, kv)
        torch.cuda.synchronize()
        assert torch.isnan(resid).all()
        assert not kd.any() and not vd.any()


def test_attention_o_rejects(gpu):
    t = torch.zeros((4096,), dtype=torch.float16, device=gpu)
    cache = torch.zeros((3, 16, 64), dtype=torch.float16, device=gpu)
    pos = torch.zeros((1,), dtype=torch.int64, device=gpu)
    inv = _inv_freq().to(gpu)
    w = torch.zeros((64, 64), dtype=torch.uint8, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="num_kv_heads"):
        _lib.attention_o_f16(t, cache, cache, inv, pos, w, t, t[:64], 6, 3)
    with pytest.raises(_lib.W4A16Error, match="head_dim"):
        _lib.attention_o_f16(t, cache, cache, inv, pos, w, t, t[:64], 4, 2, head_dim=128)
    with pytest.raises(_lib.W4A16Error, match="at most 16"):
        _lib.attention_o_f16(t, cache, cache, inv, pos, w, t, t[:64], 34, 2)


# -------------------------------- q|k|v GEMV with rotary + KV append, cached attention + o ----
def _qkv_rope_ref(x, nw, p_, s_, pos, heads, kv):
    """fp16 q|k|v rows (CPU oracle on the RMS-normalised row), then q / k rotated
    at the fp32 angle pos * inv_freq in float64 and rounded to fp16."""
    xin = _rms_norm_f16(x, nw, 1e-5) if nw is not None else x
    rows = torch.from_numpy(_f16(_linear_ref(xin, p_, s_))).to(torch.float16)
    ang = (torch.tensor(float(pos)) * _inv_freq()).double()
    c, s = ang.cos(), ang.sin()
    nq = (heads + kv) * 64
    rot = _rope64(rows[:nq].view(heads + kv, 64), c, s).to(torch.float16).reshape(-1)
    return torch.cat((rot, rows[nq:]))


@pytest.mark.parametrize("heads,kv,k", [(32, 4, 2048), (8, 2, 256), (4, 1, 5632), (16, 8, 1024)])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("pos", [0, 17, 63])
def test_gemv_qkv_rope(gpu, heads, kv, k, norm, pos):
    """qkv rows within 1e-2 (1 + |ref|) of the oracle + float64 rotation; cache
    slot pos holds the rotated k / the v rows (same bar), every other slot is
    untouched (NaN patterns included)."""
    n = (heads + 2 * kv) * 64
    S = 64
    x, p_, s_ = make_case(1, k, n, seed=pos * 7 + heads + k)
    gen = torch.Generator().manual_seed(pos + k)
    nw = (1.0 + 0.5 * torch.randn((k,), generator=gen)).to(torch.float16) if norm else None
    ref = _qkv_rope_ref(x, nw, p_, s_, pos, heads, kv)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    k_cache[:, pos + 1:] = float("nan")
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    out = torch.full((n,), float("nan"), dtype=torch.float16, device=gpu)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    print(f"[case] qkv rope heads={heads} kv={kv} K={k} norm={norm} pos={pos}", flush=True)
    _lib.gemv_qkv_rope_f16(x.to(gpu), p_.to(gpu), s_.to(gpu), out, kd, vd, _inv_freq().to(gpu), position, heads, kv,
                           norm_weight=nw.to(gpu) if norm else None, eps=1e-5)
    torch.cuda.synchronize()
    assert_parity(out.view(1, n), ref.float().numpy().reshape(1, n), f"qkv rope heads={heads} K={k}")
    kg, vg = kd.cpu(), vd.cpu()
    others = [t for t in range(S) if t != pos]
    assert torch.equal(kg[:, others].isnan(), k_cache[:, others].isnan())
    fin = [t for t in others if t < pos]
    assert torch.equal(kg[:, fin], k_cache[:, fin]) and torch.equal(vg[:, others], v_cache[:, others])
    qk = out.cpu()
    # the cache slot holds exactly what qkv holds
    assert torch.equal(kg[:, pos], qk[heads * 64: (heads + kv) * 64].view(kv, 64))
    assert torch.equal(vg[:, pos], qk[(heads + kv) * 64:].view(kv, 64))


def test_gemv_qkv_rope_position_out_of_range(gpu):
    heads, kv, k, S = 8, 2, 256, 16
    n = (heads + 2 * kv) * 64
    x, p_, s_ = make_case(1, k, n, seed=5)
    for bad in (S, -1, 1 << 40):
        kd = torch.zeros((kv, S, 64), dtype=torch.float16, device=gpu)
        vd = torch.zeros_like(kd)
        out = torch.zeros((n,), dtype=torch.float16, device=gpu)
        position = torch.tensor([bad], dtype=torch.int64, device=gpu)
        print(f"[case] qkv rope out of range pos={bad}", flush=True)
        _lib.gemv_qkv_rope_f16(x.to(gpu), p_.to(gpu), s_.to(gpu), out, kd, vd, _inv_freq().to(gpu), position,
                               heads, kv)
        torch.cuda.synchronize()
        assert not kd.any() and not vd.any()
        # the v rows are stored unrotated whatever the position
        ref = _f16(_linear_ref(x, p_, s_))[(heads + kv) * 64:]
        assert_parity(out[(heads + kv) * 64:].view(1, -1), ref.reshape(1, -1), "qkv rope v rows")


def test_gemv_qkv_rope_rejects(gpu):
    t = torch.zeros((4096,), dtype=torch.float16, device=gpu)
    cache = torch.zeros((2, 16, 64), dtype=torch.float16, device=gpu)
    pos = torch.zeros((1,), dtype=torch.int64, device=gpu)
    inv = _inv_freq().to(gpu)
    w = torch.zeros((768, 128), dtype=torch.uint8, device=gpu)
    sc = torch.zeros((768, 2), dtype=torch.float16, device=gpu)
    x = torch.zeros((256,), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="head_dim"):
        _lib.gemv_qkv_rope_f16(x, w, sc, t, cache, cache, inv, pos, 8, 2, head_dim=128)
    with pytest.raises(_lib.W4A16Error, match="group_size"):
        _lib.gemv_qkv_rope_f16(x, w, sc, t, cache, cache, inv, pos, 8, 2, group_size=64)
    with pytest.raises(_lib.W4A16Error, match="K a multiple of 128"):
        _lib.gemv_qkv_rope_f16(x[:200], w, sc, t, cache, cache, inv, pos, 8, 2)
    with pytest.raises(_lib.W4A16Error, match="aligned"):
        _lib.gemv_qkv_rope_f16(x[1:129], w, sc, t, cache, cache, inv, pos, 8, 2)


@pytest.mark.parametrize("heads,kv,hidden", [(32, 4, 2048), (8, 2, 300), (64, 8, 1000), (16, 1, 512)])
@pytest.mark.parametrize("pos", [0, 5, 47, 63])
def test_attention_o_cached(gpu, heads, kv, hidden, pos):
    """Rotated q in qkv and slot pos already in the caches (slots past pos
    NaN, which must not leak in): out = fp16(resid + fp16(o . attn)) within
    1e-2 (1 + |ref|) of the float64 attention through the CPU oracle; the
    caches are only read."""
    S = 64
    gen = torch.Generator().manual_seed(pos * 3 + hidden + heads)
    qkv = torch.randn(((heads + 2 * kv) * 64,), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    attn, k_new, v_new = _attention_ref(qkv, k_cache, v_cache, pos, heads, kv)
    ang = (torch.tensor(float(pos)) * _inv_freq()).double()
    q_rot = _rope64(qkv[: heads * 64].view(heads, 64), ang.cos(), ang.sin()).to(torch.float16).reshape(-1)
    qkv_rot = torch.cat((q_rot, torch.full(((2 * kv) * 64,), float("nan"), dtype=torch.float16)))
    k_cache[:, pos], v_cache[:, pos] = k_new, v_new
    k_cache[:, pos + 1:] = float("nan")
    v_cache[:, pos + 1:] = float("nan")
    _, op, os_ = make_case(1, heads * 64, hidden, seed=hidden + 1)
    resid = torch.randn((hidden,), generator=gen).to(torch.float16)
    ref = _f16(resid.float().numpy() + _f16(_linear_ref(attn.to(torch.float16), op, os_)))
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    out = resid.to(gpu)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    print(f"[case] attention_o cached heads={heads} kv={kv} hidden={hidden} pos={pos}", flush=True)
    _lib.attention_o_cached_f16(qkv_rot.to(gpu), kd, vd, position, op.to(gpu), os_.to(gpu), out, heads, kv)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert_parity(out.view(1, hidden), ref.reshape(1, hidden), f"attention_o cached heads={heads} hidden={hidden}")
    assert torch.equal(kd.cpu().isnan(), k_cache.isnan()) and torch.equal(vd.cpu().isnan(), v_cache.isnan())
    fin = list(range(pos + 1))
    assert torch.equal(kd.cpu()[:, fin], k_cache[:, fin]) and torch.equal(vd.cpu()[:, fin], v_cache[:, fin])


def test_attention_o_cached_position_out_of_range(gpu):
    heads, kv = 8, 2
    qkv = torch.randn(((heads + 2 * kv) * 64,)).to(torch.float16).to(gpu)
    op, os_ = _identity_o(heads * 64)
    op, os_ = op.to(gpu), os_.to(gpu)
    for S, bad in ((48, 48), (48, -1), (128, 64), (128, 100)):
        kd = torch.zeros((kv, S, 64), dtype=torch.float16, device=gpu)
        vd = torch.zeros_like(kd)
        resid = torch.zeros((heads * 64,), dtype=torch.float16, device=gpu)
        position = torch.tensor([bad], dtype=torch.int64, device=gpu)
        print(f"[case] attention_o cached out of range S={S} pos={bad}", flush=True)
        _lib.attention_o_cached_f16(qkv, kd, vd, position, op, os_, resid, heads, kv)
        torch.cuda.synchronize()
        assert torch.isnan(resid).all()
        assert not kd.any() and not vd.any()


@pytest.mark.parametrize("heads,kv,hidden", [(32, 4, 2048), (8, 2, 512)])
@pytest.mark.parametrize("pos", [3, 63])
def test_qkv_rope_pair_matches_attention_o(gpu, heads, kv, hidden, pos):
    """gemv_qkv_rope + attention_o_cached against gemv_fused + attention_o (rotary
    and append in the attention launch) on the same state: the residual rows
    within 1e-2 (1 + |ref|), cache slot pos within one fp16 rounding."""
    S, k = 64, hidden
    n = (heads + 2 * kv) * 64
    x, p_, s_ = make_case(1, k, n, seed=pos + heads)
    _, op, os_ = make_case(1, heads * 64, hidden, seed=hidden + 7)
    gen = torch.Generator().manual_seed(pos)
    nw = (1.0 + 0.5 * torch.randn((k,), generator=gen)).to(torch.float16).to(gpu)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    resid = torch.randn((hidden,), generator=gen).to(torch.float16)
    position = torch.tensor([pos], dtype=torch.int64, device=gpu)
    inv = _inv_freq().to(gpu)
    xg, pg, sg, opg, osg = x.to(gpu), p_.to(gpu), s_.to(gpu), op.to(gpu), os_.to(gpu)
    print(f"[case] qkv rope pair heads={heads} kv={kv} hidden={hidden} pos={pos}", flush=True)
    k1, v1, r1 = k_cache.to(gpu), v_cache.to(gpu), resid.to(gpu)
    qkv1 = torch.empty((n,), dtype=torch.float16, device=gpu)
    _lib.gemv_fused_f16(xg, pg, sg, qkv1, norm_weight=nw, eps=1e-5)
    _lib.attention_o_f16(qkv1, k1, v1, inv, position, opg, osg, r1, heads, kv)
    k2, v2, r2 = k_cache.to(gpu), v_cache.to(gpu), resid.to(gpu)
    qkv2 = torch.empty((n,), dtype=torch.float16, device=gpu)
    _lib.gemv_qkv_rope_f16(xg, pg, sg, qkv2, k2, v2, inv, position, heads, kv, norm_weight=nw, eps=1e-5)
    _lib.attention_o_cached_f16(qkv2, k2, v2, position, opg, osg, r2, heads, kv)
    torch.cuda.synchronize()
    assert_parity(r2.view(1, hidden), r1.float().cpu().numpy().reshape(1, hidden), "qkv rope pair")
    assert torch.equal(v2.cpu(), v1.cpu())
    assert torch.allclose(k2.cpu().float(), k1.cpu().float(), rtol=2 ** -10, atol=2 ** -14)


# ------------------------------------------------------- lm_head + argmax ----
@pytest.mark.parametrize("k,n", [(256, 1), (256, 7), (2048, 1000), (2048, 32000), (1024, 50257)])
@pytest.mark.parametrize("norm", [False, True])
def test_gemv_argmax(gpu, k, n, norm):
    """Logits bit-identical to the one-shot fused GEMV's (same arithmetic; with
    RMSNorm on 2048 x 32000 the fused GEMV takes the ring kernel, and the
    logits are checked against the oracle instead), token = torch.argmax of
    them, position + 1, embedding row gathered; three calls in a row (the
    workspace counters must return to zero)."""
    x, p, s = make_case(1, k, n, seed=k + 7 * n)
    gen = torch.Generator().manual_seed(n)
    w = (1.0 + 0.5 * torch.randn((k,), generator=gen)).to(torch.float16).to(gpu)
    xg, pg, sg = x.to(gpu).view(-1), p.to(gpu), s.to(gpu)
    ref_logits = torch.empty((n,), dtype=torch.float16, device=gpu)
    _lib.gemv_fused_f16(xg, pg, sg, ref_logits, norm_weight=w if norm else None, eps=1e-5)
    table = torch.randn((n, 96), generator=gen).to(torch.float16).to(gpu)
    ws = torch.zeros(((_lib.gemv_argmax_workspace_bytes(n) + 7) // 8,), dtype=torch.int64, device=gpu)
    token = torch.full((1,), -5, dtype=torch.int64, device=gpu)
    position = torch.tensor([10], dtype=torch.int64, device=gpu)
    for call in range(3):
        logits = torch.full((n,), float("nan"), dtype=torch.float16, device=gpu)
        emb = torch.zeros((96,), dtype=torch.float16, device=gpu)
        print(f"[case] gemv_argmax K={k} N={n} norm={norm} call {call}", flush=True)
        _lib.gemv_argmax_f16(xg, pg, sg, token, ws, logits=logits, norm_weight=w if norm else None, eps=1e-5,
                             position=position, table=table, emb_out=emb)
        torch.cuda.synchronize()
        if norm and k == 2048 and n >= 16384:
            xin = _rms_norm_f16(x, w.cpu(), 1e-5)
            assert_parity(logits.view(1, n), _linear_ref(xin, p, s).reshape(1, n), "argmax logits")
            ref_logits = logits.clone()
        assert torch.equal(logits, ref_logits)
        t = int(torch.argmax(ref_logits.float()))
        assert int(token) == t and int(position) == 11 + call
        assert torch.equal(emb, table[t])
        assert not ws[: (9 * 128) // 8].any()   # counters back at zero


def test_gemv_argmax_ties_and_no_logits(gpu):
    """Equal maxima in rows far apart: the first index wins (torch.argmax), also
    when the logits are not stored."""
    from nibble_amd.quantization import pack_int4

    k, n = 512, 20000
    x, p, s = make_case(1, k, n, seed=3)
    # rows 123, 777, 5000, 19999: codes 7 sign(x) and the largest scale, so
    # they share a logit far above every other row
    codes = torch.where(x[0] > 0, 7, -7).to(torch.int8).view(1, k)
    for r in (123, 777, 5000, 19999):
        p[r] = pack_int4(codes)[0]
        s[r] = s.max()
    xg, pg, sg = x.to(gpu).view(-1), p.to(gpu), s.to(gpu)
    logits = torch.empty((n,), dtype=torch.float16, device=gpu)
    _lib.gemv_fused_f16(xg, pg, sg, logits)
    assert float(logits.max()) == float(logits[123]) == float(logits[19999])
    ws = torch.zeros(((_lib.gemv_argmax_workspace_bytes(n) + 7) // 8,), dtype=torch.int64, device=gpu)
    token = torch.zeros((1,), dtype=torch.int64, device=gpu)
    _lib.gemv_argmax_f16(xg, pg, sg, token, ws)
    torch.cuda.synchronize()
    assert int(token) == int(torch.argmax(logits.float())) == 123


def test_gemv_argmax_rejects(gpu):
    x, p, s = make_case(1, 256, 64, seed=1)
    xg, pg, sg = x.to(gpu).view(-1), p.to(gpu), s.to(gpu)
    token = torch.zeros((1,), dtype=torch.int64, device=gpu)
    small = torch.zeros((4,), dtype=torch.int64, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="workspace"):
        _lib.gemv_argmax_f16(xg, pg, sg, token, small)
    ws = torch.zeros((1024,), dtype=torch.int64, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="both be given"):
        _lib.gemv_argmax_f16(xg, pg, sg, token, ws, table=torch.zeros((64, 8), dtype=torch.float16, device=gpu))


# ------------------------------------------------------- argmax, embedding ----
@pytest.mark.parametrize("n", [1, 1000, 32000, 50257])
def test_argmax_first_maximum_and_position(gpu, n):
    gen = torch.Generator().manual_seed(n)
    logits = torch.randn((n,), generator=gen).to(torch.float16)
    if n > 10:
        top = float(logits.max())
        logits[n // 3] = top + 1.0
        logits[n // 2] = top + 1.0        # tie: the first index wins
    token = torch.full((1,), -5, dtype=torch.int64, device=gpu)
    position = torch.tensor([41], dtype=torch.int64, device=gpu)
    _lib.argmax_f16(logits.to(gpu), token, position)
    torch.cuda.synchronize()
    assert int(token) == int(torch.argmax(logits))
    assert int(position) == 42
    _lib.argmax_f16(logits.to(gpu), token)   # no position
    torch.cuda.synchronize()
    assert int(token) == int(torch.argmax(logits))


def test_argmax_special_values(gpu):
    """The first maximum past the first round of vectors (n > 32768), in the
    scalar tail, on misaligned logits; any NaN counts as the largest value
    (the first NaN wins, in the vectors or the scalar tail, whatever its
    sign), -0 equals +0, all -inf gives token 0: each answer is torch.argmax's
    on the same logits."""
    token = torch.zeros((1,), dtype=torch.int64, device=gpu)

    def run(lg):
        _lib.argmax_f16(lg, token)
        torch.cuda.synchronize()
        got = int(token)
        assert got == int(torch.argmax(lg.float().cpu())), (got, int(torch.argmax(lg.float().cpu())))
        return got

    gen = torch.Generator().manual_seed(5)
    lg = torch.randn((40000,), generator=gen).to(torch.float16)
    lg[39000] = 9.0
    lg[39001] = 9.0
    assert run(lg.to(gpu)) == 39000
    lg[12345] = 9.0                       # the same maximum in the first round wins
    assert run(lg.to(gpu)) == 12345
    lg[33000] = float("nan")              # a NaN beats every number
    assert run(lg.to(gpu)) == 33000
    lg[100] = -float("nan")               # the first NaN wins, whatever its sign
    assert run(lg.to(gpu)) == 100
    tail = torch.zeros((33,), dtype=torch.float16)
    tail[32] = 5.0                        # index 32 is past the 4 vectors
    assert run(tail.to(gpu)) == 32
    tail[7] = 5.0
    assert run(tail.to(gpu)) == 7
    buf = torch.zeros((34,), dtype=torch.float16, device=gpu)
    buf[1:] = tail.to(gpu)
    assert run(buf[1:]) == 7              # misaligned: every element on the scalar path
    buf[30] = float("nan")
    assert run(buf[1:]) == 29             # a NaN on the scalar path
    tail[32] = float("nan")
    tail[7] = 5.0
    assert run(tail.to(gpu)) == 32        # a NaN in the vectors' scalar tail
    zeros = torch.zeros((100,), dtype=torch.float16)
    zeros[:50] = -0.0
    assert run(zeros.to(gpu)) == 0        # -0 equals +0: the first index
    assert run(torch.full((1000,), float("-inf"), dtype=torch.float16, device=gpu)) == 0
    neg = torch.full((1000,), float("-inf"), dtype=torch.float16)
    neg[600] = -60000.0
    assert run(neg.to(gpu)) == 600
    neg[10] = float("nan")
    assert run(neg.to(gpu)) == 10


@pytest.mark.parametrize("hidden", [2048, 8200, 4100, 24])
def test_argmax_embed_gathers_next_row(gpu, hidden):
    """The row is gathered by 16-byte vectors (several per lane past 512
    halves) or, for a hidden size that is not a multiple of 8 or a
    misaligned output, element by element."""
    vocab = 1000
    table = torch.randn((vocab, hidden)).to(torch.float16).to(gpu)
    logits = torch.randn((vocab,)).to(torch.float16)
    logits[777] = 50.0
    token = torch.zeros((1,), dtype=torch.int64, device=gpu)
    position = torch.tensor([3], dtype=torch.int64, device=gpu)
    out = torch.zeros((hidden,), dtype=torch.float16, device=gpu)
    _lib.argmax_embed_f16(logits.to(gpu), token, position, table, out)
    torch.cuda.synchronize()
    assert int(token) == 777 and int(position) == 4
    assert torch.equal(out, table[777])
    # misaligned logits take the scalar path
    buf = torch.empty((vocab + 1,), dtype=torch.float16, device=gpu)
    buf[1:] = logits.to(gpu)
    _lib.argmax_embed_f16(buf[1:], token, None, table, out)
    torch.cuda.synchronize()
    assert int(token) == 777
    # misaligned output: element by element
    obuf = torch.zeros((hidden + 1,), dtype=torch.float16, device=gpu)
    _lib.argmax_embed_f16(logits.to(gpu), token, None, table, obuf[1:])
    torch.cuda.synchronize()
    assert torch.equal(obuf[1:], table[777]) and float(obuf[0]) == 0.0
    # the token history slot: only that element is written
    history = torch.full((4,), -1, dtype=torch.int64, device=gpu)
    _lib.argmax_embed_f16(logits.to(gpu), token, position, table, out, token_copy=history[2:3])
    torch.cuda.synchronize()
    assert history.tolist() == [-1, -1, 777, -1] and int(token) == 777 and int(position) == 5


def test_embedding_gather(gpu):
    table = torch.randn((100, 2048)).to(torch.float16).to(gpu)
    out = torch.empty((2048,), dtype=torch.float16, device=gpu)
    for t in (0, 57, 99):
        _lib.embedding_f16(table, torch.tensor([t], device=gpu), out)
        torch.cuda.synchronize()
        assert torch.equal(out, table[t])
    _lib.embedding_f16(table, torch.tensor([100], device=gpu), out)
    torch.cuda.synchronize()
    assert not out.any()


# ----------------------------------------------------------- fused decoder ----
def _small_cfg():
    from nibble_amd.llama import LlamaConfig

    return LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1280, num_layers=2, num_heads=8,
                       num_kv_heads=2, head_dim=64, max_seq_len=32)


def test_fused_step_matches_torch_step(gpu):
    """One decode step from the same state: fused kernels vs the torch-op step
    around QuantizedLinear (same weights). Bar on the logits:
    |err| <= 2e-2 (1 + |ref|)."""
    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(_small_cfg(), device=gpu, seed=0)
    assert model.fused
    prompt = torch.randint(0, 512, (12,), generator=torch.Generator().manual_seed(1)).to(gpu)
    model.prefill(prompt)
    state = (model.k_cache.clone(), model.v_cache.clone(), model.token.clone(), model.position.clone())
    with torch.inference_mode():
        model.fused = False
        model.step()
        ref_logits, ref_k = model.logits.clone(), model.k_cache.clone()
        model.k_cache.copy_(state[0]); model.v_cache.copy_(state[1])
        model.token.copy_(state[2]); model.position.copy_(state[3])
        model.fused = True
        model.step()
    torch.cuda.synchronize()
    got, ref = model.logits.float().cpu(), ref_logits.float().cpu()
    assert torch.all((got - ref).abs() <= 2e-2 * (1 + ref.abs())), float((got - ref).abs().max())
    assert int(model.position) == int(state[3]) + 1
    # the new cache slot holds the same k (rotary within fp16 rounding)
    p = int(state[3])
    assert torch.allclose(model.k_cache[:, :, p].float(), ref_k[:, :, p].float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("size,bound", [("small", 5e-3), ("full", 2e-2)])
def test_decoder_matches_cpu_reference_path(gpu, size, bound):
    """The GPU decoder (fused prefill, fused decode step with attention + o)
    against the same weights on the CPU, where every projection runs the
    product's torch restatement of the reference's path (dequantize, fp32
    matmul: nibble_amd.reference, pinned against the C oracle in
    tests/test_api_cpu.py) and attention, RMSNorm and SiLU are torch ops: the
    prefill's last-position logits and one decode step's logits within
    bound * (1 + |ref|) (small model: measured 1.5e-3 at |ref| <= 1.65), on
    the 2-layer test model and on configs[4] at full size (22 layers,
    hidden 2048, 155 INT4 linears, 16-token prompt). No HIP code on the
    reference side."""
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = _small_cfg() if size == "small" else LlamaConfig(max_seq_len=48)
    model = LlamaDecoder(cfg, device=gpu, seed=0)
    ref = LlamaDecoder(cfg, device="cpu", init="empty")
    ref.load_state_dict({k: v.detach().cpu() for k, v in model.state_dict().items()})
    assert model.fused and model.attn_o and not ref.fused
    prompt = torch.randint(0, cfg.vocab_size, (12 if size == "small" else 16,),
                           generator=torch.Generator().manual_seed(5))
    with torch.inference_mode():
        print("[case] decoder vs CPU reference path: prefill", flush=True)
        model.prefill(prompt.to(gpu))
        torch.cuda.synchronize()
        got = model.logits.float().cpu()
        ref.k_cache.zero_()
        ref.v_cache.zero_()
        want = ref._forward(prompt, torch.arange(prompt.numel())).float()
        assert torch.isfinite(got).all()
        print(f"[case] {size}: prefill logits max |err| {float((got - want).abs().max()):.3e}", flush=True)
        assert torch.all((got - want).abs() <= bound * (1 + want.abs())), float((got - want).abs().max())
        # the CPU model's state for the step, and the same next token on the
        # GPU (a near-tie in the argmax must not change the comparison)
        ref.prefill(prompt)
        model.token.copy_(ref.token.to(gpu))
        model.x_buf.copy_(model.embed[model.token[0]])
        print("[case] decoder vs CPU reference path: one step", flush=True)
        model.step()
        ref.step()
        torch.cuda.synchronize()
        got, want = model.logits.float().cpu(), ref.logits.float()
        print(f"[case] {size}: step logits max |err| {float((got - want).abs().max()):.3e}", flush=True)
        assert torch.all((got - want).abs() <= bound * (1 + want.abs())), float((got - want).abs().max())
        assert int(model.position) == int(ref.position) == prompt.numel() + 1


def test_attention_o_step_matches_two_launch_step(gpu):
    """From the same state, the step with attention + o as one launch and the
    step with separate attention and o GEMV launches agree (logits
    |err| <= 2e-2 (1 + |ref|), same new token, same cache slot within fp16
    rounding)."""
    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(_small_cfg(), device=gpu, seed=4)
    assert model.attn_o
    prompt = torch.randint(0, 512, (20,), generator=torch.Generator().manual_seed(9)).to(gpu)
    model.prefill(prompt)
    state = (model.k_cache.clone(), model.v_cache.clone(), model.token.clone(), model.position.clone(),
             model.x_buf.clone())
    with torch.inference_mode():
        model._step(short=False)
        ref_logits, ref_k, ref_tok = model.logits.clone(), model.k_cache.clone(), model.token.clone()
        for t, s in zip((model.k_cache, model.v_cache, model.token, model.position, model.x_buf), state):
            t.copy_(s)
        model._step(short=True)
    torch.cuda.synchronize()
    got, ref = model.logits.float().cpu(), ref_logits.float().cpu()
    assert torch.all((got - ref).abs() <= 2e-2 * (1 + ref.abs())), float((got - ref).abs().max())
    assert torch.equal(model.token, ref_tok)
    p = int(state[3])
    assert torch.allclose(model.k_cache[:, :, p].float(), ref_k[:, :, p].float(), rtol=1e-2, atol=1e-2)


def test_split_attention_step(gpu):
    """A 640-slot cache takes the split decode attention (5 shares per head):
    from the same state after a 600-token prompt, the fused step against the
    torch-op step and against the fused step with one workgroup per head
    (logits |err| <= 2e-2 (1 + |ref|)); graphed tokens equal eager ones."""
    from dataclasses import replace

    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(replace(_small_cfg(), max_seq_len=640), device=gpu, seed=5)
    assert model.attn_splits == 5
    prompt = torch.randint(0, 512, (600,), generator=torch.Generator().manual_seed(6)).to(gpu)
    model.prefill(prompt)
    state = (model.k_cache.clone(), model.v_cache.clone(), model.token.clone(), model.position.clone(),
             model.x_buf.clone())

    def step(fused: bool, splits: int):
        for t, s_ in zip((model.k_cache, model.v_cache, model.token, model.position, model.x_buf), state):
            t.copy_(s_)
        model.fused, model.attn_splits = fused, splits
        with torch.inference_mode():
            model.step()
        torch.cuda.synchronize()
        return model.logits.float().cpu(), model.k_cache.clone()

    ref, ref_k = step(False, 5)
    got, got_k = step(True, 5)
    one, _ = step(True, 0)
    for other in (ref, one):
        assert torch.all((got - other).abs() <= 2e-2 * (1 + other.abs())), float((got - other).abs().max())
    assert torch.allclose(got_k[:, :, 600].float(), ref_k[:, :, 600].float(), rtol=1e-2, atol=1e-2)
    model.attn_splits = 5
    eager = model.generate(prompt, 6, use_graph=False)
    model.prefill(prompt)
    model.capture()
    assert torch.equal(model.generate(prompt, 6, use_graph=True), eager)


def test_decode_graphs_across_position_64(gpu):
    """Generation that crosses position 64 switches from the attention + o
    graph to the general one; graph replays equal eager decode (which switches
    at the same step)."""
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1280, num_layers=2, num_heads=8,
                      num_kv_heads=2, head_dim=64, max_seq_len=96)
    model = LlamaDecoder(cfg, device=gpu, seed=11)
    prompt = torch.randint(0, 512, (58,), generator=torch.Generator().manual_seed(12)).to(gpu)
    eager = model.generate(prompt, 12, use_graph=False)
    model.prefill(prompt)
    model.capture()
    assert model.graph_short is not None
    assert torch.equal(model.generate(prompt, 12, use_graph=True), eager)
    assert model.host_position == 58 + 11 and int(model.position) == 58 + 11


def test_fused_decode_graph_matches_eager(gpu):
    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(_small_cfg(), device=gpu, seed=2)
    prompt = torch.randint(0, 512, (10,), generator=torch.Generator().manual_seed(3)).to(gpu)
    eager = model.generate(prompt, 10, use_graph=False)
    model.prefill(prompt)
    model.capture()
    for _ in range(2):
        assert torch.equal(model.generate(prompt, 10, use_graph=True), eager)


@pytest.mark.parametrize("tokens_per_replay", [2, 4, 7])
def test_multi_step_graph_matches_eager(gpu, tokens_per_replay):
    """Several decode steps per graph replay (capture(tokens_per_replay=T)):
    the same tokens as eager decode, and as one step per replay; prompts that
    leave the graph's range (position 64) fall back to single steps."""
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1280, num_layers=2, num_heads=8,
                      num_kv_heads=2, head_dim=64, max_seq_len=80)
    model = LlamaDecoder(cfg, device=gpu, seed=5)
    for plen, new in ((10, 20), (50, 25)):
        prompt = torch.randint(0, 512, (plen,), generator=torch.Generator().manual_seed(plen)).to(gpu)
        print(f"[case] multi-step T={tokens_per_replay} prompt={plen} new={new}", flush=True)
        eager = model.generate(prompt, new, use_graph=False)
        model.prefill(prompt)
        model.capture()
        single = model.generate(prompt, new, use_graph=True)
        model.prefill(prompt)
        model.capture(tokens_per_replay=tokens_per_replay)
        assert model.graph_multi is not None
        multi = model.generate(prompt, new, use_graph=True)
        assert torch.equal(single, eager)
        assert torch.equal(multi, eager)


def test_full_size_fused_step_and_graphed_tokens(gpu):
    """configs[4] at full size (22 layers, hidden 2048, 155 INT4 linears, the
    benchmark's seeds): one fused decode step against the torch-op step from
    the same state (logits |err| <= 2e-2 (1 + |ref|)), and 32 greedy tokens
    from HIP-graph replays equal to eager fused decode."""
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(max_seq_len=48)
    model = LlamaDecoder(cfg, device=gpu, seed=0)
    assert model.fused and model.attn_o and len(model.linear_layers()) == 155
    prompt = torch.randint(0, cfg.vocab_size, (16,), generator=torch.Generator().manual_seed(0)).to(gpu)
    print("[case] full-size 1.1B: prefill + one step each path", flush=True)
    model.prefill(prompt)
    state = (model.k_cache.clone(), model.v_cache.clone(), model.token.clone(), model.position.clone(),
             model.x_buf.clone())
    with torch.inference_mode():
        model.fused = False
        model.step()
        ref_logits = model.logits.clone()
        for t, s in zip((model.k_cache, model.v_cache, model.token, model.position, model.x_buf), state):
            t.copy_(s)
        model.fused = True
        model.host_position = int(state[3])
        model.step()
    torch.cuda.synchronize()
    got, ref = model.logits.float().cpu(), ref_logits.float().cpu()
    assert torch.isfinite(got).all()
    assert torch.all((got - ref).abs() <= 2e-2 * (1 + ref.abs())), float((got - ref).abs().max())
    print("[case] full-size 1.1B: 32 tokens eager vs graph", flush=True)
    eager = model.generate(prompt, 32, use_graph=False)
    model.prefill(prompt)
    model.capture()
    graphed = model.generate(prompt, 32, use_graph=True)
    assert graphed.shape == (32,) and torch.equal(graphed, eager)


def test_checkpoint_into_fused_decoder(gpu, tmp_path):
    """A whole-model checkpoint (reference format) from an offline Hugging Face
    Llama with head_dim 64 runs on the fused step: graph replays equal eager
    fused decode, and the first fused step's logits match the torch-op step."""
    transformers = pytest.importorskip("transformers")
    from nibble_amd import model_checkpoint as mc

    cfg = transformers.LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, rms_norm_eps=1e-5,
                                   max_position_embeddings=64, tie_word_embeddings=False)
    torch.manual_seed(5)
    try:
        hf = transformers.AutoModelForCausalLM.from_config(cfg, dtype=torch.float16)
    except TypeError:
        hf = transformers.AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.float16)
    mc.quantize_model(hf, 128)
    ckpt = mc.load_model_checkpoint(mc.save_model_checkpoint(hf, tmp_path / "m.pt", "t", 128))
    dec = mc.decoder_from_checkpoint(ckpt, mc.decoder_config(cfg.to_dict(), max_seq_len=32), device=gpu)
    assert dec.fused
    prompt = torch.randint(0, 512, (8,), generator=torch.Generator().manual_seed(6)).to(gpu)
    eager = dec.generate(prompt, 6, use_graph=False)
    dec.prefill(prompt)
    dec.capture()
    assert torch.equal(dec.generate(prompt, 6, use_graph=True), eager)


@pytest.mark.parametrize("tokens", [16, 40])
def test_native_and_graphed_prefill(gpu, tokens):
    """Torch-op prefill with the W4A16 op for the projections (16 tokens: the
    one-shot MFMA kernel; 40: the GEMM; fused q|k|v and gate|up) matches the
    dequantize + hipBLASLt module path (logits |err| <= 2e-2 (1 + |ref|)),
    and the graphed prefill reproduces the eager one exactly."""
    from dataclasses import replace

    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(replace(_small_cfg(), max_seq_len=64), device=gpu, seed=7)
    model.fuse_prefill = False   # prefill() takes the torch-op path checked here
    prompt = torch.randint(0, 512, (tokens,), generator=torch.Generator().manual_seed(8)).to(gpu)
    positions = torch.arange(tokens, device=gpu)
    with torch.inference_mode():
        for b in model.layers:
            b.native_prefill = False
        model.k_cache.zero_(); model.v_cache.zero_()
        ref = model._forward(prompt, positions).float()
        for b in model.layers:
            b.native_prefill = True
        model.k_cache.zero_(); model.v_cache.zero_()
        got = model._forward(prompt, positions).float()
    assert torch.all((got - ref).abs() <= 2e-2 * (1 + ref.abs())), float((got - ref).abs().max())
    eager_tok = model.prefill(prompt)
    k_eager, x_eager = model.k_cache.clone(), model.x_buf.clone()
    model.capture_prefill(tokens)
    other = torch.randint(0, 512, (tokens,), generator=torch.Generator().manual_seed(9)).to(gpu)
    model.prefill(other)                       # a replay on different tokens in between
    assert torch.equal(model.prefill(prompt), eager_tok)
    assert torch.equal(model.k_cache, k_eager) and torch.equal(model.x_buf, x_eager)
    assert int(model.position) == tokens
