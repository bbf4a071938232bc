"""GPU tests of the prefill launches (include/w4a16_decode.h: RMSNorm rows,
SiLU * up, prefill attention) against float64 / torch restatements, and of
the decoder's fused prefill against its torch-op prefill."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from nibble_amd import _lib

pytestmark = pytest.mark.gpu

ULP = 2.0 ** -10   # one fp16 unit in the last place, relative


def _tables(S: int, theta: float = 10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, 64, 2).float() / 64))
    ang = torch.outer(torch.arange(S).float(), inv)
    return ang.cos(), ang.sin()


def _rope64(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    x1, x2 = x[..., :32].double(), x[..., 32:].double()
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


@pytest.mark.parametrize("rows,hidden", [(1, 2048), (16, 2048), (7, 5632), (3, 100)])
def test_rmsnorm_rows(gpu, rows, hidden):
    gen = torch.Generator().manual_seed(rows * 7 + hidden)
    x = (3.0 * torch.randn((rows, hidden), generator=gen)).to(torch.float16)
    w = (1.0 + 0.5 * torch.randn((hidden,), generator=gen)).to(torch.float16)
    eps = 1e-5
    xd = x.double()
    ref = (xd * torch.rsqrt(xd.pow(2).mean(dim=-1, keepdim=True) + eps)) * w.double()
    out = torch.full((rows, hidden), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] rmsnorm rows={rows} hidden={hidden}", flush=True)
    _lib.rmsnorm_f16(x.to(gpu), w.to(gpu), eps, out)
    torch.cuda.synchronize()
    got = out.double().cpu()
    # one fp16 rounding of a value within fp32 error of the exact one
    assert torch.all((got - ref).abs() <= ULP * ref.abs() + 2 ** -24), float((got - ref).abs().max())


@pytest.mark.parametrize("rows,hidden", [(16, 2048), (1, 2048), (5, 8192), (3, 24)])
def test_embed_rmsnorm_rows(gpu, rows, hidden):
    """w4a16_embed_rmsnorm_f16: the gathered rows exactly, the norm bit-identical
    to w4a16_rmsnorm_f16 on the gathered rows (and within one fp16 rounding of
    float64), zeros for a token outside the table, position <- rows."""
    vocab = 300
    gen = torch.Generator().manual_seed(rows + hidden)
    table = (2.0 * torch.randn((vocab, hidden), generator=gen)).to(torch.float16).to(gpu)
    w = (1.0 + 0.5 * torch.randn((hidden,), generator=gen)).to(torch.float16).to(gpu)
    tokens = torch.randint(0, vocab, (rows,), generator=gen)
    if rows > 2:
        tokens[1] = vocab + 5   # out of range: a zero row
        tokens[2] = tokens[0]   # a repeated token
    tokens = tokens.to(gpu)
    eps = 1e-5
    x = torch.full((rows, hidden), float("nan"), dtype=torch.float16, device=gpu)
    out = torch.full((rows, hidden), float("nan"), dtype=torch.float16, device=gpu)
    position = torch.tensor([-7], dtype=torch.int64, device=gpu)
    print(f"[case] embed + rmsnorm rows={rows} hidden={hidden}", flush=True)
    _lib.embed_rmsnorm_f16(table, tokens, w, eps, x, out, position=position)
    gathered = torch.zeros((rows, hidden), dtype=torch.float16, device=gpu)
    ok = (tokens >= 0) & (tokens < vocab)
    gathered[ok] = table[tokens[ok]]
    ref = torch.empty_like(out)
    _lib.rmsnorm_f16(gathered, w, eps, ref)
    torch.cuda.synchronize()
    assert torch.equal(x, gathered)
    assert torch.equal(out, ref)
    assert int(position) == rows
    gd = gathered.double().cpu()
    exact = (gd * torch.rsqrt(gd.pow(2).mean(dim=-1, keepdim=True) + eps)) * w.double().cpu()
    got = out.double().cpu()
    assert torch.all((got - exact).abs() <= ULP * exact.abs() + 2 ** -24), float((got - exact).abs().max())


@pytest.mark.parametrize("rows,hidden,alias", [(1, 2048, True), (64, 2048, True), (7, 5632, False), (3, 100, False),
                                              (2, 8192, True)])
def test_add_rmsnorm_rows(gpu, rows, hidden, alias):
    """x_out = x + delta with the rounding of an fp16 tensor add (bit-exact
    against torch), output = RMSNorm(x_out) * w within one fp16 rounding of
    float64; x_out may be x itself."""
    gen = torch.Generator().manual_seed(rows * 3 + hidden)
    x = (3.0 * torch.randn((rows, hidden), generator=gen)).to(torch.float16)
    d = (2.0 * torch.randn((rows, hidden), generator=gen)).to(torch.float16)
    w = (1.0 + 0.5 * torch.randn((hidden,), generator=gen)).to(torch.float16)
    eps = 1e-5
    s_ref = (x.float() + d.float()).to(torch.float16)
    sd = s_ref.double()
    ref = (sd * torch.rsqrt(sd.pow(2).mean(dim=-1, keepdim=True) + eps)) * w.double()
    xd, dd = x.to(gpu), d.to(gpu)
    x_out = xd if alias else torch.full_like(xd, float("nan"))
    out = torch.full((rows, hidden), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] add_rmsnorm rows={rows} hidden={hidden} alias={alias}", flush=True)
    _lib.add_rmsnorm_f16(xd, dd, w.to(gpu), eps, x_out, out)
    torch.cuda.synchronize()
    assert torch.equal(x_out.cpu(), s_ref)
    got = out.double().cpu()
    assert torch.all((got - ref).abs() <= ULP * ref.abs() + 2 ** -24), float((got - ref).abs().max())
    # w4a16_rmsnorm_f16 on the sum agrees to one fp16 rounding (measured: 7
    # of 131072 outputs one ulp apart at 64 x 2048; the two launches' fp32
    # normalisers can differ in the last bit)
    plain = torch.empty_like(out)
    _lib.rmsnorm_f16(s_ref.to(gpu), w.to(gpu), eps, plain)
    torch.cuda.synchronize()
    pf = plain.double().cpu()
    assert torch.all((pf - got).abs() <= ULP * pf.abs()), float((pf - got).abs().max())


def test_add_rmsnorm_rejects(gpu):
    x = torch.zeros((2, 8200), dtype=torch.float16, device=gpu)
    w = torch.ones((8200,), dtype=torch.float16, device=gpu)
    out = torch.zeros_like(x)
    with pytest.raises(_lib.W4A16Error, match="8192"):
        _lib.add_rmsnorm_f16(x, x, w, 1e-5, x, out)


@pytest.mark.parametrize("rows,inter", [(1, 5632), (16, 5632), (5, 77), (64, 5632), (3, 40)])
def test_silu_mul(gpu, rows, inter):
    gen = torch.Generator().manual_seed(rows + inter)
    gu = (4.0 * torch.randn((rows, 2 * inter), generator=gen)).to(torch.float16)
    g, u = gu[:, :inter].double(), gu[:, inter:].double()
    silu16 = (g / (1 + torch.exp(-g))).to(torch.float16).double()
    ref = silu16 * u
    out = torch.full((rows, inter), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] silu_mul rows={rows} inter={inter}", flush=True)
    _lib.silu_mul_f16(gu.to(gpu), out)
    torch.cuda.synchronize()
    got = out.double().cpu()
    # silu(g) within one fp16 ulp of the exact rounding, then one more rounding
    assert torch.all((got - ref).abs() <= 3 * ULP * ref.abs() + 2 ** -20), float((got - ref).abs().max())
    # and against torch's own fp16 ops on the same tensors
    torch_ref = (F.silu(gu[:, :inter].to(gpu)) * gu[:, inter:].to(gpu)).double().cpu()
    assert torch.all((got - torch_ref).abs() <= 2 * ULP * torch_ref.abs() + 2 ** -20)


@pytest.mark.parametrize("m,k,inter", [(1, 2048, 5632), (2, 2048, 5632), (16, 2048, 5632), (9, 2048, 5000),
                                       (13, 5632, 1000), (12, 2048, 4100), (64, 2048, 5632),
                                       (37, 1152, 100), (1, 20480, 64), (130, 4096, 257), (256, 2048, 5632),
                                       (128, 5632, 2100)])
def test_linear_silu(gpu, m, k, inter, monkeypatch):
    """w4a16_linear_silu_f16 against the op over the 2 inter rows followed by
    SiLU * up: bit-identical to the same GEMM shape (or, at M = 1 with K <=
    16384, to the paired fused GEMV), and within the parity bar of the oracle's
    fp32 products pushed through the same fp16 roundings."""
    from tests._cases import expected, make_case

    x, p, s = make_case(m, k, 2 * inter, seed=m + k + inter)
    xd, pd, sd = x.to(gpu), p.to(gpu), s.to(gpu)
    out = torch.full((m, inter), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] linear_silu M={m} K={k} inter={inter}", flush=True)
    _lib.linear_silu_f16(xd, pd, sd, out)
    gu = torch.empty((m, 2 * inter), dtype=torch.float16, device=gpu)
    ref16 = None
    if m == 1 and k <= 16384:
        _lib.gemv_fused_f16(xd[0], pd, sd, out_ref := torch.empty((inter,), dtype=torch.float16, device=gpu),
                            paired=True)
        ref = out_ref.view(1, inter)
    else:
        # M = 9..16 on rows longer than 4096 weights or on wide layers of rows
        # up to 2048: the 16-row-slot paired kernel's SiLU form where its plan
        # stages whole rows (else the GEMM's); its sibling is the plain 16-slot
        # kernel over the 2 inter rows (selector mfma_pair), same K split,
        # same sums
        # M = 9..16 on rows of 2048 weights of wide layers: the paired ring
        # kernel's SiLU form, whose sibling is its plain 16-slot form with
        # the same K split (four wavefronts of 2 pairs each, their sums added
        # in order) over the 2 inter rows
        ring16 = 9 <= m <= 16 and k == 2048 and 2 * inter >= 8192
        silu16 = 9 <= m <= 16 and (k > 4096 or (k <= 2048 and 2 * inter >= 8192))
        if ring16:
            _lib.linear_f16_tuned(xd, pd, sd, gu, 128, _lib.KERNEL_PAIR_RING, 2, 4, 2)
            ref16 = torch.empty_like(out)
            _lib.silu_mul_f16(gu, ref16)
        elif silu16:
            monkeypatch.setenv("W4A16_DECODE", "mfma_pair")
            _lib.linear_f16(xd, pd, sd, gu)
            monkeypatch.delenv("W4A16_DECODE")
            ref16 = torch.empty_like(out)
            _lib.silu_mul_f16(gu, ref16)
        # the same GEMM over the 2 inter rows (the op's shape), then SiLU * up
        monkeypatch.setenv("W4A16_DECODE", "valu")   # for M > 8: off the paired and one-shot MFMA routes
        plan = _lib.plan_linear(1 << 20, 1 << 20, m, 2 * inter, k, 128)
        monkeypatch.delenv("W4A16_DECODE")
        # the SiLU form of the 32x32 kernel: the first of 128, 64, 32 output
        # columns per workgroup (K split 1, 2, 4 ways) with >= 160 workgroups;
        # the plain 32x32 GEMM with the same K split sums in the same order
        silu32 = [sk for cols, sk in ((128, 1), (64, 2), (32, 4))
                  if m >= 64 and k <= 4096 and -(-inter // cols) * -(-m // 64) >= 160]
        if silu32:
            rows, unroll = {1: (4, 4), 2: (2, 4), 4: (2, 2)}[silu32[0]]
            _lib.linear_f16_tuned(xd, pd, sd, gu, 128, _lib.KERNEL_GEMM32, rows, silu32[0], unroll, 1)
        elif plan["kernel"] == "gemm_lds":
            _lib.linear_f16_tuned(xd, pd, sd, gu, 128, _lib.KERNEL_GEMM_LDS, 4, plan["splits"], plan["unroll"], 2)
        elif plan["kernel"] == "gemm":
            _lib.linear_f16_tuned(xd, pd, sd, gu, 128, _lib.KERNEL_GEMM, plan["rows"], plan["splits"], 0, 2)
        else:   # M = 1, K > 16384: the op runs a GEMV; compare with the GEMM at 1 activation tile
            _lib.linear_f16_tuned(xd, pd, sd, gu, 128, _lib.KERNEL_GEMM, 1, 4, 0, 2)
        ref = torch.empty_like(out)
        _lib.silu_mul_f16(gu, ref)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    if 9 <= m <= 16 and k == 2048 and 2 * inter >= 8192:   # the 1.1B decoder's gate|up: the ring SiLU form
        assert torch.equal(out, ref16)
    elif ref16 is None or not torch.equal(out, ref16):
        assert torch.equal(out, ref)
    g = torch.from_numpy(expected(x, p, s)).to(torch.float16).double()   # the op's fp16 outputs (oracle)
    sg = (g[:, :inter] / (1 + torch.exp(-g[:, :inter]))).to(torch.float16).double()
    want = sg * g[:, inter:]
    got = out.double().cpu()
    assert torch.all((got - want).abs() <= 1e-2 * (1 + want.abs())), float((got - want).abs().max())


def _prefill_attention_ref(qkv, k_cache, v_cache, cos, sin, start, heads, kv):
    """float64 restatement: rotary q / k rounded to fp16, causal softmax attention."""
    t = qkv.shape[0]
    slots = torch.arange(start, start + t)
    c, s = cos[slots].double().unsqueeze(1), sin[slots].double().unsqueeze(1)
    q = _rope64(qkv[:, : heads * 64].view(t, heads, 64), c, s).to(torch.float16)
    k_new = _rope64(qkv[:, heads * 64: (heads + kv) * 64].view(t, kv, 64), c, s).to(torch.float16)
    v_new = qkv[:, (heads + kv) * 64:].view(t, kv, 64)
    kc, vc = k_cache.clone(), v_cache.clone()
    kc[:, start: start + t] = k_new.transpose(0, 1)
    vc[:, start: start + t] = v_new.transpose(0, 1)
    group = heads // kv
    nk = start + t
    kf = kc.double().repeat_interleave(group, 0)[:, :nk]            # [heads, nk, 64]
    vf = vc.double().repeat_interleave(group, 0)[:, :nk]
    qd = q.double().transpose(0, 1)                                  # [heads, t, 64]
    scores = torch.matmul(qd, kf.transpose(1, 2)) / math.sqrt(64)   # [heads, t, nk]
    mask = torch.arange(nk).unsqueeze(0) > (start + torch.arange(t)).unsqueeze(1)
    scores = scores.masked_fill(mask, float("-inf"))
    out = torch.matmul(torch.softmax(scores, dim=-1), vf)           # [heads, t, 64]
    return out.transpose(0, 1).reshape(t, heads * 64), kc, vc, k_new, v_new


_ATTN_CASES = [(1, 0), (5, 0), (16, 0), (64, 0), (16, 7), (64, 192), (7, 3), (130, 0), (256, 0), (100, 101)]


@pytest.mark.parametrize("heads,kv,misaligned", [(32, 4, False), (8, 8, False), (4, 1, False), (32, 1, False),
                                                 (64, 1, False), (12, 4, False), (32, 4, True)])
@pytest.mark.parametrize("tokens,start", _ATTN_CASES)
def test_prefill_attention(gpu, heads, kv, misaligned, tokens, start):
    """Query heads per KV head a power of two up to 64 with 16-byte aligned
    qkv and tables: the matrix-core kernel (64 query columns per workgroup);
    otherwise (group 3, or qkv at a 2-byte offset) the one-query-per-wavefront
    kernels."""
    S = 256
    gen = torch.Generator().manual_seed(tokens * 13 + start + heads + kv)
    qkv = torch.randn((tokens, (heads + 2 * kv) * 64), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    cos, sin = _tables(S)
    ref, kc_ref, vc_ref, k_new, v_new = _prefill_attention_ref(qkv, k_cache, v_cache, cos, sin, start, heads, kv)
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    out = torch.full((tokens, heads * 64), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] prefill attention heads={heads} kv={kv} tokens={tokens} start={start} misaligned={misaligned}",
          flush=True)
    if misaligned:
        buf = torch.empty((qkv.numel() + 1,), dtype=torch.float16, device=gpu)
        buf[1:] = qkv.to(gpu).view(-1)
        qkv_d = buf[1:].view(qkv.shape)
    else:
        qkv_d = qkv.to(gpu)
    _lib.prefill_attention_f16(qkv_d, kd, vd, cos.to(gpu), sin.to(gpu), start, out, heads, kv)
    torch.cuda.synchronize()
    got = out.double().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert torch.all(err <= 2e-3 + 1e-2 * ref.abs()), float(err.max())
    # caches: slots start .. start + tokens - 1 replaced (v exact, rotary k within an fp16 ulp), others untouched
    kg, vg = kd.cpu(), vd.cpu()
    new = slice(start, start + tokens)
    others = [s for s in range(S) if not start <= s < start + tokens]
    assert torch.equal(kg[:, others], k_cache[:, others]) and torch.equal(vg[:, others], v_cache[:, others])
    assert torch.equal(vg[:, new], v_new.transpose(0, 1))
    assert torch.allclose(kg[:, new].float(), k_new.transpose(0, 1).float(), rtol=ULP, atol=2 ** -14)


# past the 256 slots LDS holds at once: the new rows appended by their own
# launch, the caches streamed through LDS in blocks of 256 slots (1 to 3
# blocks, a partial last block, a start past the first block)
@pytest.mark.parametrize("heads,kv", [(32, 4), (8, 8), (64, 1)])
@pytest.mark.parametrize("tokens,start,S", [(257, 0, 320), (300, 0, 512), (100, 300, 512), (520, 0, 1024),
                                            (64, 700, 1024)])
def test_prefill_attention_streamed(gpu, heads, kv, tokens, start, S):
    gen = torch.Generator().manual_seed(tokens * 7 + start + heads)
    qkv = torch.randn((tokens, (heads + 2 * kv) * 64), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    cos, sin = _tables(S)
    ref, kc_ref, vc_ref, k_new, v_new = _prefill_attention_ref(qkv, k_cache, v_cache, cos, sin, start, heads, kv)
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    out = torch.full((tokens, heads * 64), float("nan"), dtype=torch.float16, device=gpu)
    print(f"[case] streamed prefill attention heads={heads} kv={kv} tokens={tokens} start={start} S={S}", flush=True)
    _lib.prefill_attention_f16(qkv.to(gpu), kd, vd, cos.to(gpu), sin.to(gpu), start, out, heads, kv)
    torch.cuda.synchronize()
    got = out.double().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert torch.all(err <= 2e-3 + 1e-2 * ref.abs()), float(err.max())
    kg, vg = kd.cpu(), vd.cpu()
    new = slice(start, start + tokens)
    others = [s for s in range(S) if not start <= s < start + tokens]
    assert torch.equal(kg[:, others], k_cache[:, others]) and torch.equal(vg[:, others], v_cache[:, others])
    assert torch.equal(vg[:, new], v_new.transpose(0, 1))
    assert torch.allclose(kg[:, new].float(), k_new.transpose(0, 1).float(), rtol=ULP, atol=2 ** -14)


def test_prefill_attention_rejects(gpu):
    heads, kv, S = 8, 2, 300
    kd = torch.zeros((kv, S, 64), dtype=torch.float16, device=gpu)
    vd = torch.zeros_like(kd)
    cos, sin = _tables(S)
    cos, sin = cos.to(gpu), sin.to(gpu)
    short_k = torch.zeros((kv, 64, 64), dtype=torch.float16, device=gpu)
    for tokens, start, kc, vc in [(301, 0, kd, vd), (10, 295, kd, vd), (10, 60, short_k, short_k)]:
        # past the caches' 300 (or 64) slots
        qkv = torch.zeros((tokens, (heads + 2 * kv) * 64), dtype=torch.float16, device=gpu)
        out = torch.zeros((tokens, heads * 64), dtype=torch.float16, device=gpu)
        with pytest.raises(_lib.W4A16Error, match="tokens"):
            _lib.prefill_attention_f16(qkv, kc, vc, cos, sin, start, out, heads, kv)
    # past 256 slots only the matrix-core layout streams: not group 3, not qkv at a 2-byte offset
    for h, misaligned in [(6, False), (8, True)]:
        buf = torch.zeros((257 * (h + 2 * kv) * 64 + 1,), dtype=torch.float16, device=gpu)
        qkv = (buf[1:] if misaligned else buf[:-1]).view(257, (h + 2 * kv) * 64)
        out = torch.zeros((257, h * 64), dtype=torch.float16, device=gpu)
        with pytest.raises(_lib.W4A16Error, match="256 slots"):
            _lib.prefill_attention_f16(qkv, kd, vd, cos, sin, 0, out, h, kv)
    qkv = torch.zeros((4, (heads + 2 * kv) * 64), dtype=torch.float16, device=gpu)
    out = torch.zeros((4, heads * 64), dtype=torch.float16, device=gpu)
    with pytest.raises(_lib.W4A16Error, match="head_dim"):
        _lib.prefill_attention_f16(qkv, kd, vd, cos, sin, 0, out, heads, kv, head_dim=128)
    with pytest.raises(_lib.W4A16Error, match="multiple"):
        _lib.prefill_attention_f16(qkv, kd, vd, cos, sin, 0, out, 7, 2)
    assert not kd.any() and not vd.any()


def _small_cfg():
    from nibble_amd.llama import LlamaConfig

    return LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1280, num_layers=2, num_heads=8,
                       num_kv_heads=2, head_dim=64, max_seq_len=32)


@pytest.mark.parametrize("tokens", [1, 9, 16, 17, 33, 64, 130, 300, 600, 1100])
def test_fused_prefill_matches_torch_prefill(gpu, tokens):
    """The fused prefill (up to 16 tokens the one-shot / paired MFMA kernels,
    beyond that the GEMM; from 300 tokens the attention streams through
    256-slot blocks, and 1100 tokens take dequantize + hipBLASLt projections)
    against the torch-op prefill of the same model and prompt: logits of the
    last token within 2e-2 (1 + |ref|), KV caches within fp16 roundings; the
    graphed fused prefill reproduces the eager one exactly."""
    from dataclasses import replace

    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(replace(_small_cfg(), max_seq_len=max(160, tokens + 16)), device=gpu, seed=11)
    prompt = torch.randint(0, 512, (tokens,), generator=torch.Generator().manual_seed(tokens)).to(gpu)
    assert model.fused_prefill(tokens)
    with torch.inference_mode():
        model.k_cache.zero_(); model.v_cache.zero_()
        ref = model._forward(prompt, torch.arange(tokens, device=gpu)).float()
        k_ref, v_ref = model.k_cache.clone().float(), model.v_cache.clone().float()
    tok = model.prefill(prompt)
    got = model.logits.float()
    assert torch.all((got - ref).abs() <= 2e-2 * (1 + ref.abs())), float((got - ref).abs().max())
    assert torch.allclose(model.k_cache.float(), k_ref, rtol=1e-2, atol=1e-2)
    assert torch.allclose(model.v_cache.float(), v_ref, rtol=1e-2, atol=1e-2)
    assert int(model.position) == tokens
    assert torch.equal(model.x_buf, model.embed[tok[0]])
    logits_eager, k_eager = model.logits.clone(), model.k_cache.clone()
    model.capture_prefill(tokens)
    other = torch.randint(0, 512, (tokens,), generator=torch.Generator().manual_seed(99)).to(gpu)
    model.prefill(other)
    assert torch.equal(model.prefill(prompt), tok)
    assert torch.equal(model.logits, logits_eager) and torch.equal(model.k_cache, k_eager)


@pytest.mark.parametrize("tokens", [16, 33, 70])
def test_fused_prefill_ignores_stale_cache_slots(gpu, tokens):
    """The fused prefill does not reset the KV caches: slots past the prompt
    keep what they held, and every fused attention kernel (the prompt's, the
    short step's attention + o launch, the split attention past 64) selects
    them away. With NaN in every slot beforehand, the greedy tokens of the
    prefill and 6 decode steps and the caches' prompt slots equal those of a
    run on zeroed caches, eager and with the prefill graph."""
    from dataclasses import replace

    from nibble_amd.llama import LlamaDecoder

    model = LlamaDecoder(replace(_small_cfg(), max_seq_len=tokens + 8), device=gpu, seed=5)
    prompt = torch.randint(0, 512, (tokens,), generator=torch.Generator().manual_seed(tokens + 1)).to(gpu)
    assert model.fused_prefill(tokens)
    print(f"[case] stale cache slots, {tokens}-token prompt", flush=True)
    with torch.inference_mode():
        model.k_cache.zero_(); model.v_cache.zero_()
    ref = model.generate(prompt, 7, use_graph=False)
    k_ref, v_ref = model.k_cache[:, :, :tokens].clone(), model.v_cache[:, :, :tokens].clone()
    assert not bool(torch.isnan(model.logits).any())
    for graphed in (False, True):
        with torch.inference_mode():
            model.k_cache.fill_(float("nan")); model.v_cache.fill_(float("nan"))
        if graphed:
            model.capture_prefill(tokens)
            with torch.inference_mode():
                model.k_cache.fill_(float("nan")); model.v_cache.fill_(float("nan"))
        got = model.generate(prompt, 7, use_graph=False)
        assert torch.equal(got, ref), (graphed, got.tolist(), ref.tolist())
        assert torch.equal(model.k_cache[:, :, :tokens], k_ref) and torch.equal(model.v_cache[:, :, :tokens], v_ref)
        assert bool(torch.isnan(model.k_cache[:, :, tokens + 6:]).all())


# (query heads, KV heads, tokens, start, hidden): 9..16 tokens at slots up to
# 31 with K = 2048 and a power-of-two group take the attention inside the o
# op's launch (configs[4]'s prompt first; slots below start from the caches;
# group 4, 8 and 32; hidden 1024); past slot 31, at 8 tokens, on K = 1024,
# group 3 and hidden 2000 the separate launches
_ATTN_O_CASES = [(32, 4, 16, 0, 2048), (32, 4, 9, 0, 2048), (32, 4, 12, 7, 2048), (32, 4, 16, 16, 2048),
                 (32, 8, 16, 0, 1024), (32, 1, 13, 3, 2048), (32, 4, 16, 17, 2048), (32, 4, 8, 0, 2048),
                 (16, 4, 16, 0, 2048), (12, 4, 16, 0, 1024), (32, 4, 16, 0, 2000)]


@pytest.mark.parametrize("heads,kv,tokens,start,hidden", _ATTN_O_CASES)
def test_prefill_attention_o_add_rmsnorm_matches_separate_launches(gpu, heads, kv, tokens, start, hidden):
    """w4a16_prefill_attention_o_add_rmsnorm_f16 against the prefill
    attention, the op and the residual add + RMSNorm as three launches: the
    v cache bit for bit, the rotary k rows within an fp16 ulp (each kernel
    rounds its fp32 rotation to fp16, the compiler choosing a single fused
    rounding or fp32 then fp16 per instruction), x_out (in place) and the
    normed rows within a few fp16 ulps; the separate launches' attention rows
    are held to the float64 restatement and their o op to the oracle."""
    from tests._cases import assert_parity, expected, make_case

    S = 64
    k = heads * 64
    gen = torch.Generator().manual_seed(heads * 100 + kv * 10 + tokens + start + hidden)
    qkv = torch.randn((tokens, (heads + 2 * kv) * 64), generator=gen).to(torch.float16)
    k_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    v_cache = torch.randn((kv, S, 64), generator=gen).to(torch.float16)
    cos, sin = _tables(S)
    _, p, s = make_case(tokens, k, hidden, seed=hidden + tokens)
    resid = torch.randn((tokens, hidden), generator=gen).to(torch.float16)
    w = (1 + 0.1 * torch.randn((hidden,), generator=gen)).to(torch.float16)
    qkv_d, cos_d, sin_d = qkv.to(gpu), cos.to(gpu), sin.to(gpu)
    pd, sd, wd, resid_d = p.to(gpu), s.to(gpu), w.to(gpu), resid.to(gpu)
    print(f"[case] prefill attention + o + add_rmsnorm heads={heads} kv={kv} tokens={tokens} start={start} "
          f"hidden={hidden}", flush=True)
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    x = resid_d.clone()
    h = torch.full((tokens, hidden), float("nan"), dtype=torch.float16, device=gpu)
    _lib.prefill_attention_o_add_rmsnorm_f16(qkv_d, kd, vd, cos_d, sin_d, start, pd, sd, x, wd, 1e-5, x, h, heads,
                                             kv)
    # the separate launches
    ks, vs = k_cache.to(gpu), v_cache.to(gpu)
    attn = torch.empty((tokens, k), dtype=torch.float16, device=gpu)
    _lib.prefill_attention_f16(qkv_d, ks, vs, cos_d, sin_d, start, attn, heads, kv)
    d = torch.empty((tokens, hidden), dtype=torch.float16, device=gpu)
    _lib.linear_f16(attn, pd, sd, d)
    xs, hs = torch.empty_like(resid_d), torch.empty_like(h)
    _lib.add_rmsnorm_f16(resid_d, d, wd, 1e-5, xs, hs)
    torch.cuda.synchronize()
    assert torch.equal(vd, vs)
    assert torch.allclose(kd.float(), ks.float(), rtol=ULP, atol=2 ** -14)
    for got, want, name in ((x, xs, "x_out"), (h, hs, "normed rows")):
        err = (got.float() - want.float()).abs()
        assert torch.all(err <= 4e-3 + 4 * ULP * want.float().abs()), (name, float(err.max()))
    ref = _prefill_attention_ref(qkv, k_cache, v_cache, cos, sin, start, heads, kv)[0]
    err = (attn.double().cpu() - ref).abs()
    assert torch.all(err <= 2e-3 + 1e-2 * ref.abs()), float(err.max())
    assert_parity(d, expected(attn.cpu(), p, s), f"o op tokens={tokens} K={k} N={hidden}")


@pytest.mark.parametrize("m,k,n,alias", [(16, 5632, 2048, True), (12, 5632, 2048, False), (9, 5632, 2048, True),
                                         (16, 14336, 4096, False), (4, 5632, 2048, False), (16, 8192, 2048, True),
                                         (16, 5632, 2044, False), (13, 5632, 1000, True)])
def test_linear_add_rmsnorm_matches_separate_launches(gpu, m, k, n, alias):
    """w4a16_linear_add_rmsnorm_f16 against the op with a workspace followed
    by w4a16_add_rmsnorm_f16, bit for bit: where the op takes the ring
    kernel's K slices on rows of at most 2048 outputs (M >= 12 on 5632 and
    8192, N a multiple of 8) the slices are summed in the norm's launch,
    elsewhere (other M, 4096 outputs, N not a multiple of 8) the two launches
    run as they are; x_out in place or apart."""
    from tests._cases import assert_parity, expected, make_case

    x16, p, s = make_case(m, k, n, seed=m + k + n)
    a, pd, sd = x16.to(gpu), p.to(gpu), s.to(gpu)
    gen = torch.Generator().manual_seed(n)
    resid = torch.randn((m, n), generator=gen).to(torch.float16).to(gpu)
    w = (1 + 0.1 * torch.randn((n,), generator=gen)).to(torch.float16).to(gpu)
    print(f"[case] linear_add_rmsnorm M={m} K={k} N={n} alias={alias}", flush=True)
    xin = resid.clone()
    x_out = xin if alias else torch.full_like(resid, float("nan"))
    h = torch.full((m, n), float("nan"), dtype=torch.float16, device=gpu)
    _lib.linear_add_rmsnorm_f16(a, pd, sd, xin, w, 1e-5, x_out, h)
    # the separate launches
    d = torch.empty((m, n), dtype=torch.float16, device=gpu)
    _lib.linear_f16(a, pd, sd, d)
    xs = torch.empty_like(resid)
    hs = torch.empty_like(h)
    _lib.add_rmsnorm_f16(resid, d, w, 1e-5, xs, hs)
    torch.cuda.synchronize()
    assert torch.equal(x_out, xs)
    assert torch.equal(h, hs)
    assert_parity(d, expected(x16, p, s), f"linear M={m} K={k} N={n}")
