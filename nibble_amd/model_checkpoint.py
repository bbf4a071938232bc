"""Whole-model W4A16 checkpoints, built and read offline.

File format -- a ``torch.save`` dict, the layout of the reference's
TinyLlama checkpoint (``scripts/quantize_tinyllama.py:71-83``) so files made
by either side load on the other:

    {"format": "w4a16-tinyllama", "version": 1, "source_model": str,
     "group_size": int, "state_dict": {key: CPU tensor}}

where ``state_dict`` is a Hugging Face Llama state dict after
``replace_linear_layers`` (``*.packed_weights`` / ``*.scales`` for every
quantized linear, fp16 tensors for the rest). Loading uses
``torch.load(weights_only=True)`` and the reference's checks and messages
(``scripts/generate.py:214-226``).

Besides the reference's two steps (quantize a model and save; load into a
model skeleton), this module maps such a checkpoint onto
``nibble_amd.llama.LlamaDecoder``, so a locally stored Llama model runs on
the fused decode step.

Command line (no network: ``--model`` is a local Hugging Face directory, or
``--random-init`` builds the architecture from a config):

    python -m nibble_amd.model_checkpoint quantize --output ckpt.pt \\
        (--model DIR | --random-init [--config tinyllama|tiny] [--seed 0]) [--group-size 128]
    python -m nibble_amd.model_checkpoint validate ckpt.pt
"""

from __future__ import annotations

import argparse
import re
import sys
import warnings
from pathlib import Path

import torch

from nibble_amd.integration import load_packed_state_dict, replace_linear_layers

CHECKPOINT_FORMAT = "w4a16-tinyllama"
CHECKPOINT_VERSION = 1

# Llama-architecture configs the command line can build without a download.
CONFIGS = {
    # TinyLlama-1.1B's architecture (the reference's decode model)
    "tinyllama": dict(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=22,
                      num_attention_heads=32, num_key_value_heads=4, rms_norm_eps=1e-5, rope_theta=10000.0,
                      max_position_embeddings=2048, tie_word_embeddings=False),
    "tiny": dict(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                 num_attention_heads=4, num_key_value_heads=2, rms_norm_eps=1e-5, rope_theta=10000.0,
                 max_position_embeddings=128, tie_word_embeddings=False),
}


# ------------------------------------------------------------- quantize/save --
def quantize_model(model: torch.nn.Module, group_size: int = 128) -> int:
    """Swap every compatible ``nn.Linear`` for a ``QuantizedLinear`` in place
    (reference ``scripts/quantize_tinyllama.py:55-66``); returns the count.
    Skipped layers are reported as ``UserWarning``s."""
    if group_size <= 0:
        raise ValueError("group_size must be greater than zero")
    with torch.inference_mode():
        return replace_linear_layers(model, group_size=group_size)


def save_model_checkpoint(model: torch.nn.Module, path: str | Path, source_model: str, group_size: int) -> Path:
    """Write the whole-model dict (reference ``scripts/quantize_tinyllama.py:71-83``)."""
    out = Path(path)
    out.parent.mkdir(parents=True, exist_ok=True)
    torch.save(
        {
            "format": CHECKPOINT_FORMAT,
            "version": CHECKPOINT_VERSION,
            "source_model": source_model,
            "group_size": group_size,
            "state_dict": {key: tensor.detach().cpu() for key, tensor in model.state_dict().items()},
        },
        out,
    )
    return out


# ------------------------------------------------------------------- load ----
def load_model_checkpoint(path: str | Path) -> dict:
    """Read and validate a whole-model checkpoint (reference
    ``scripts/generate.py:214-226``: same checks, same messages)."""
    checkpoint = torch.load(Path(path), map_location="cpu", weights_only=True)
    if not isinstance(checkpoint, dict):
        raise ValueError("checkpoint must contain a dictionary")
    if checkpoint.get("format") != CHECKPOINT_FORMAT:
        raise ValueError("checkpoint has an unsupported format")
    if checkpoint.get("version") != CHECKPOINT_VERSION:
        raise ValueError("checkpoint has an unsupported version")
    if not isinstance(checkpoint.get("group_size"), int):
        raise ValueError("checkpoint is missing group_size")
    if not isinstance(checkpoint.get("state_dict"), dict):
        raise ValueError("checkpoint is missing state_dict")
    return checkpoint


def load_packed_model(model: torch.nn.Module, checkpoint: dict, device: str | torch.device = "cpu",
                      fused: bool = True) -> int:
    """Load a validated checkpoint into a model skeleton (``nn.Linear`` layers,
    e.g. built on the meta device): linears become ``QuantizedLinear`` holding
    the packed tensors, without materialising fp16 weights (reference
    ``scripts/generate.py:229-257``). Returns the number of replaced layers."""
    return load_packed_state_dict(model, checkpoint["state_dict"], group_size=checkpoint["group_size"],
                                  device=device, fused=fused)


# ------------------------------------------------- onto the fused decoder ----
_LAYER_KEYS = {
    "input_layernorm.weight": "input_norm.weight",
    "post_attention_layernorm.weight": "post_norm.weight",
    "self_attn.q_proj": "q_proj",
    "self_attn.k_proj": "k_proj",
    "self_attn.v_proj": "v_proj",
    "self_attn.o_proj": "o_proj",
    "mlp.gate_proj": "gate_proj",
    "mlp.up_proj": "up_proj",
    "mlp.down_proj": "down_proj",
}


def hf_to_decoder_state_dict(state_dict: dict, group_size: int = 128) -> dict:
    """Rename a Hugging Face Llama state dict (after quantization) to
    ``LlamaDecoder``'s keys. An fp16 ``lm_head.weight`` (an lm_head left
    unquantized) is quantized here with the same RTN rule; a tied lm_head
    (no ``lm_head.*`` key) is quantized from the embedding. Buffers HF
    recomputes (``rotary_emb.inv_freq``) are dropped; any other key raises."""
    from nibble_amd.quantization import quantize_and_pack_weights

    out: dict = {}
    for key, value in state_dict.items():
        if key == "model.embed_tokens.weight":
            out["embed"] = value
        elif key == "model.norm.weight":
            out["norm.weight"] = value
        elif key in ("lm_head.packed_weights", "lm_head.scales"):
            out[key] = value
        elif key == "lm_head.weight":
            out["lm_head.packed_weights"], out["lm_head.scales"] = quantize_and_pack_weights(value, group_size)
        elif key.endswith("rotary_emb.inv_freq"):
            continue
        else:
            m = re.fullmatch(r"model\.layers\.(\d+)\.(.+?)(\.packed_weights|\.scales|)$", key)
            name = None
            if m:
                layer, rest, suffix = m.groups()
                base = _LAYER_KEYS.get(rest)
                if base is not None:
                    name = f"layers.{layer}.{base}{suffix}"
            if name is None:
                raise KeyError(f"checkpoint key '{key}' has no place in LlamaDecoder "
                               "(unquantized linear weight, bias, or not a Llama model)")
            out[name] = value
    if "lm_head.packed_weights" not in out and "embed" in out:
        out["lm_head.packed_weights"], out["lm_head.scales"] = quantize_and_pack_weights(out["embed"], group_size)
    return out


def decoder_config(hf_config: dict, max_seq_len: int = 2048):
    """``LlamaConfig`` of ``nibble_amd.llama`` from a Hugging Face Llama config dict."""
    from nibble_amd.llama import LlamaConfig

    heads = hf_config["num_attention_heads"]
    return LlamaConfig(
        vocab_size=hf_config["vocab_size"], hidden_size=hf_config["hidden_size"],
        intermediate_size=hf_config["intermediate_size"], num_layers=hf_config["num_hidden_layers"],
        num_heads=heads, num_kv_heads=hf_config.get("num_key_value_heads", heads),
        head_dim=hf_config.get("head_dim") or hf_config["hidden_size"] // heads,
        rms_norm_eps=hf_config.get("rms_norm_eps", 1e-6), rope_theta=hf_config.get("rope_theta", 10000.0),
        max_seq_len=max_seq_len,
    )


def decoder_from_checkpoint(checkpoint: dict, config, device: str | torch.device = "cuda", fused: bool = True):
    """A ``LlamaDecoder`` holding the checkpoint's weights (group size from the
    checkpoint; ``config`` is a ``nibble_amd.llama.LlamaConfig``)."""
    from nibble_amd.llama import LlamaDecoder

    if checkpoint["group_size"] != config.group_size:
        config.group_size = checkpoint["group_size"]
    model = LlamaDecoder(config, device=device, fused=fused, init="empty")
    state = hf_to_decoder_state_dict(checkpoint["state_dict"], config.group_size)
    missing, unexpected = model.load_state_dict(state, strict=False)
    if missing or unexpected:
        raise KeyError(f"checkpoint does not match the decoder: missing {sorted(missing)[:5]}, "
                       f"unexpected {sorted(unexpected)[:5]}")
    return model


# ------------------------------------------------------------ command line --
def _build_hf_model(args):
    import transformers

    if args.model:
        model = transformers.AutoModelForCausalLM.from_pretrained(args.model, torch_dtype=torch.float16,
                                                                  local_files_only=True)
        return model, args.model
    cfg = transformers.LlamaConfig(**CONFIGS[args.config])
    torch.manual_seed(args.seed)
    model = transformers.AutoModelForCausalLM.from_config(cfg, torch_dtype=torch.float16)
    return model, f"random-init:{args.config}:seed{args.seed}"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m nibble_amd.model_checkpoint", description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    q = sub.add_parser("quantize", help="quantize a local or random-init Llama model and save the checkpoint")
    src = q.add_mutually_exclusive_group(required=True)
    src.add_argument("--model", help="local Hugging Face model directory (no download)")
    src.add_argument("--random-init", action="store_true", help="build the architecture of --config")
    q.add_argument("--config", choices=sorted(CONFIGS), default="tinyllama")
    q.add_argument("--seed", type=int, default=0)
    q.add_argument("--group-size", type=int, default=128)
    q.add_argument("--device", choices=["cpu", "cuda"], default="cpu")
    q.add_argument("--output", required=True)
    v = sub.add_parser("validate", help="check a checkpoint and summarise it")
    v.add_argument("path")
    args = ap.parse_args(argv)

    if args.cmd == "quantize":
        if args.group_size <= 0:
            raise ValueError("group_size must be greater than zero")
        model, source = _build_hf_model(args)
        model = model.to(args.device).eval()
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always", UserWarning)
            count = quantize_model(model, args.group_size)
        print(f"replacement_count: {count}")
        for w in caught:
            if issubclass(w.category, UserWarning):
                print(w.message)
        print(f"wrote {save_model_checkpoint(model, args.output, source, args.group_size)}")
        return 0

    ckpt = load_model_checkpoint(args.path)
    sd = ckpt["state_dict"]
    packed = [k for k in sd if k.endswith(".packed_weights")]
    nbytes = sum(sd[k].numel() for k in packed) + sum(sd[k[: -len("packed_weights")] + "scales"].numel() * 2
                                                        for k in packed)
    print(f"format {ckpt['format']} v{ckpt['version']}, source {ckpt.get('source_model')}, "
          f"group_size {ckpt['group_size']}: {len(packed)} packed linears, {nbytes} packed bytes, "
          f"{len(sd)} tensors")
    return 0


if __name__ == "__main__":
    sys.exit(main())
