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
