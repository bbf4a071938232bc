"""Whole-model checkpoint tooling (nibble_amd.model_checkpoint), on the CPU:
the reference's TinyLlama checkpoint format (scripts/quantize_tinyllama.py:71-83)
and validator (scripts/generate.py:214-226), built from an offline Hugging
Face Llama, and the mapping onto the fused decoder."""

from __future__ import annotations

import pytest
import torch

from nibble_amd import model_checkpoint as mc
from nibble_amd.linear import QuantizedLinear

transformers = pytest.importorskip("transformers")

TINY = dict(vocab_size=96, hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, rms_norm_eps=1e-5, rope_theta=10000.0, max_position_embeddings=64,
            tie_word_embeddings=False)


def _hf_model(seed: int = 0, **overrides):
    cfg = transformers.LlamaConfig(**{**TINY, **overrides})
    torch.manual_seed(seed)
    try:
        model = transformers.AutoModelForCausalLM.from_config(cfg, dtype=torch.float16)
    except TypeError:
        model = transformers.AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.float16)
    # non-trivial norm weights, so the RMSNorm weight path is exercised
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_((1.0 + 0.2 * torch.randn_like(p.float())).to(p.dtype))
    return model.eval(), cfg


def test_quantize_save_load_round_trip(tmp_path):
    model, cfg = _hf_model()
    assert mc.quantize_model(model, 128) == 2 * 7 + 1
    path = mc.save_model_checkpoint(model, tmp_path / "m.pt", "random-init:test", 128)
    ckpt = mc.load_model_checkpoint(path)
    assert ckpt["format"] == "w4a16-tinyllama" and ckpt["version"] == 1 and ckpt["group_size"] == 128
    assert ckpt["source_model"] == "random-init:test"

    with torch.device("meta"):
        try:
            skeleton = transformers.AutoModelForCausalLM.from_config(cfg, dtype=torch.float16)
        except TypeError:
            skeleton = transformers.AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.float16)
    assert mc.load_packed_model(skeleton, ckpt, device="cpu") == 15
    assert isinstance(skeleton.model.layers[0].self_attn.q_proj, QuantizedLinear)
    for key, value in model.state_dict().items():
        assert torch.equal(skeleton.state_dict()[key], value), key
    ids = torch.randint(0, cfg.vocab_size, (1, 7), generator=torch.Generator().manual_seed(1))
    with torch.inference_mode():
        assert torch.equal(model(ids).logits, skeleton.eval()(ids).logits)


@pytest.mark.parametrize(
    "mutate,message",
    [
        (lambda c: "not a dict", "must contain a dictionary"),
        (lambda c: {**c, "format": "other"}, "unsupported format"),
        (lambda c: {**c, "version": 2}, "unsupported version"),
        (lambda c: {k: v for k, v in c.items() if k != "group_size"}, "missing group_size"),
        (lambda c: {**c, "state_dict": [1, 2]}, "missing state_dict"),
    ],
)
def test_validator_rejects(tmp_path, mutate, message):
    good = {"format": "w4a16-tinyllama", "version": 1, "source_model": "x", "group_size": 128,
            "state_dict": {"a": torch.zeros(1)}}
    torch.save(mutate(good), tmp_path / "bad.pt")
    with pytest.raises(ValueError, match=message):
        mc.load_model_checkpoint(tmp_path / "bad.pt")


def test_decoder_from_checkpoint_matches_hf(tmp_path):
    """The fused decoder (its CPU torch-op path here) on the checkpoint's
    weights reproduces the quantized Hugging Face model's next-token logits
    (same INT4 weights; RMSNorm, rotary and attention rounding orders differ
    slightly between the two: bar |err| <= 2e-2 (1 + |ref|))."""
    from nibble_amd.llama import LlamaDecoder

    model, cfg = _hf_model(seed=3)
    mc.quantize_model(model, 128)
    ckpt = mc.load_model_checkpoint(mc.save_model_checkpoint(model, tmp_path / "m.pt", "t", 128))
    dcfg = mc.decoder_config(cfg.to_dict(), max_seq_len=32)
    dec = mc.decoder_from_checkpoint(ckpt, dcfg, device="cpu")
    assert isinstance(dec, LlamaDecoder) and len(dec.linear_layers()) == 15
    prompt = torch.randint(0, cfg.vocab_size, (9,), generator=torch.Generator().manual_seed(2))
    with torch.inference_mode():
        ref = model(prompt.view(1, -1)).logits[0, -1].float()
        positions = torch.arange(prompt.numel())
        dec.k_cache.zero_()
        dec.v_cache.zero_()
        got = dec._forward(prompt, positions).float()
    assert torch.all((got - ref).abs() <= 2e-2 * (1 + ref.abs())), float((got - ref).abs().max())
    assert int(torch.argmax(got)) == int(torch.argmax(ref))


def test_state_dict_mapping_edges():
    model, _ = _hf_model(seed=4)
    mc.quantize_model(model, 128)
    sd = model.state_dict()
    mapped = mc.hf_to_decoder_state_dict(sd)
    assert torch.equal(mapped["layers.1.gate_proj.packed_weights"], sd["model.layers.1.mlp.gate_proj.packed_weights"])
    assert torch.equal(mapped["layers.0.post_norm.weight"], sd["model.layers.0.post_attention_layernorm.weight"])
    # tied / unquantized lm_head: quantized from the fp16 matrix with the same RTN rule
    from nibble_amd.quantization import quantize_and_pack_weights

    no_head = {k: v for k, v in sd.items() if not k.startswith("lm_head")}
    tied = mc.hf_to_decoder_state_dict(no_head)
    p, s = quantize_and_pack_weights(sd["model.embed_tokens.weight"], 128)
    assert torch.equal(tied["lm_head.packed_weights"], p) and torch.equal(tied["lm_head.scales"], s)
    with pytest.raises(KeyError, match="no place in LlamaDecoder"):
        mc.hf_to_decoder_state_dict({**sd, "model.layers.0.self_attn.q_proj.bias": torch.zeros(128)})


def test_command_line(tmp_path, capsys):
    out = tmp_path / "tiny.pt"
    assert mc.main(["quantize", "--random-init", "--config", "tiny", "--output", str(out)]) == 0
    assert "replacement_count: 15" in capsys.readouterr().out
    assert mc.main(["validate", str(out)]) == 0
    text = capsys.readouterr().out
    assert "w4a16-tinyllama v1" in text and "15 packed linears" in text
