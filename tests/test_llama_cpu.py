"""The Llama decode model's structure on the CPU path (tiny config): layer
count, greedy decode determinism, and that decoding with a KV cache gives
the same next token as re-running the whole prefix."""

from __future__ import annotations

import torch

from nibble_amd.llama import LlamaConfig, LlamaDecoder


def _tiny():
    return LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=256, num_layers=2, num_heads=4,
                       num_kv_heads=2, head_dim=32, max_seq_len=16)


def test_layer_count_and_bytes():
    cfg = LlamaConfig()
    assert cfg.num_linear_layers == 155
    m = LlamaDecoder(_tiny(), device="cpu")
    assert len(m.linear_layers()) == 2 * 7 + 1


def test_kv_cache_decode_equals_full_recompute():
    m = LlamaDecoder(_tiny(), device="cpu", seed=3)
    prompt = torch.randint(0, 64, (5,), generator=torch.Generator().manual_seed(0))
    toks = m.generate(prompt, 4, use_graph=False)
    # recompute each next token from scratch on the growing sequence
    seq = prompt.clone()
    for i in range(4):
        nxt = m.prefill(seq)
        assert int(nxt) == int(toks[i])
        seq = torch.cat([seq, nxt])


def test_fused_weight_buffers_keep_state_dict_layout():
    """q|k|v and gate|up rows live in one buffer each; every module's
    packed_weights / scales is a contiguous view of its own rows, so the
    state dict keeps the per-module keys and shapes."""
    cfg = _tiny()
    m = LlamaDecoder(cfg, device="cpu", seed=1)
    sd = m.state_dict()
    kv = cfg.num_kv_heads * cfg.head_dim
    for i, b in enumerate(m.layers):
        assert sd[f"layers.{i}.q_proj.packed_weights"].shape == (cfg.hidden_size, cfg.hidden_size // 2)
        assert sd[f"layers.{i}.k_proj.packed_weights"].shape == (kv, cfg.hidden_size // 2)
        assert sd[f"layers.{i}.up_proj.scales"].shape == (cfg.intermediate_size, cfg.hidden_size // 128)
        qkv_w, qkv_s = m.qkv[i]
        gu_w, gu_s = m.gate_up[i]
        assert qkv_w.shape[0] == cfg.hidden_size + 2 * kv and gu_w.shape[0] == 2 * cfg.intermediate_size
        for mod in (b.q_proj, b.k_proj, b.v_proj, b.gate_proj, b.up_proj):
            assert mod.packed_weights.is_contiguous() and mod.scales.is_contiguous()
        assert b.k_proj.packed_weights.data_ptr() == qkv_w[cfg.hidden_size:].data_ptr()
        assert b.v_proj.scales.data_ptr() == qkv_s[cfg.hidden_size + kv:].data_ptr()
        assert b.up_proj.packed_weights.data_ptr() == gu_w[cfg.intermediate_size:].data_ptr()
        assert torch.equal(torch.cat([b.gate_proj.packed_weights, b.up_proj.packed_weights]), gu_w)
    assert not m.fused   # the fused step runs on GPUs only


def test_prefill_length_and_split_attention_rules():
    """Host-side routing of the decoder: the fused prefill takes any prompt
    that fits the cache when query heads per KV head are a power of two up to
    64 (the attention streams the caches), else prompts up to 256 tokens; the
    decode attention splits over the slots only past 512 cache slots, into
    256 / heads shares, with a workspace of heads * shares * 66 fp32."""
    from dataclasses import replace

    from nibble_amd.llama import FUSED_PREFILL_MAX_TOKENS

    streamed = LlamaDecoder(replace(_tiny(), max_seq_len=600), device="cpu")
    streamed.fused = True   # the fused path's host rules, without a GPU
    assert streamed.fused_prefill(1) and streamed.fused_prefill(300) and streamed.fused_prefill(600)
    assert not streamed.fused_prefill(0) and not streamed.fused_prefill(601)
    streamed.fuse_prefill = False
    assert not streamed.fused_prefill(16)
    odd = LlamaDecoder(replace(_tiny(), num_heads=12, num_kv_heads=4, hidden_size=12 * 32, max_seq_len=600),
                       device="cpu")
    odd.fused = True
    assert odd.fused_prefill(FUSED_PREFILL_MAX_TOKENS) and not odd.fused_prefill(FUSED_PREFILL_MAX_TOKENS + 1)
    assert streamed.attn_splits == min(256 // 4, 600 // 128) == 4
    assert streamed.attn_ws.numel() == 4 * 4 * 66
    assert LlamaDecoder(replace(_tiny(), max_seq_len=512), device="cpu").attn_splits == 0
    # few query heads and a long cache: capped at the split launch's 64 shares
    few = replace(_tiny(), num_heads=2, num_kv_heads=2, max_seq_len=16384)
    assert LlamaDecoder(few, device="cpu").attn_splits == 64
