"""The reference's Python API through the drop-in import name ``w4a16`` (CPU
tensors): the reference's own unit tests -- known values, round trips,
errors, routing, model patching, meta-device loading, checkpoints -- restated
for this package (reference tests/test_quantization.py, test_reference.py,
test_checkpoint.py, test_linear.py, test_integration.py), plus agreement of
the product's CPU path with the oracle."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

import oracle
import w4a16
from w4a16.checkpoint import load_quantized_weight_checkpoint, save_quantized_weight_checkpoint
from w4a16.integration import load_packed_state_dict, replace_linear_layers
from w4a16.linear import FUSED_MAX_ROWS, Int4Linear, QuantizedLinear
from w4a16.quantization import pack_int4, quantize_and_pack_weights, quantize_groupwise, unpack_int4
from w4a16.reference import dequantize_weights, linear_reference

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


def t16(a):
    return torch.tensor(a, dtype=torch.float16)


# ------------------------------------------------------------ package ----
def test_public_names():
    for name in ["QuantizedLinear", "pack_int4", "unpack_int4", "quantize_groupwise", "quantize_and_pack_weights",
                 "save_quantized_weight_checkpoint", "load_quantized_weight_checkpoint", "replace_linear_layers",
                 "load_packed_state_dict", "linear_cuda", "dequantize_cuda", "cuda_extension_available"]:
        assert hasattr(w4a16, name), name
    assert Int4Linear is QuantizedLinear
    assert FUSED_MAX_ROWS == 8
    import importlib

    assert importlib.import_module("w4a16._C") is importlib.import_module("nibble_amd._C")


# ------------------------------------------------------- quantization ----
def test_pack_known_values():
    assert torch.equal(pack_int4(torch.tensor(KAT["pack_int4"]["codes"], dtype=torch.int8)),
                       torch.tensor(KAT["pack_int4"]["packed"], dtype=torch.uint8))


def test_unpack_known_values():
    assert torch.equal(unpack_int4(torch.tensor(KAT["unpack_int4"]["packed"], dtype=torch.uint8)),
                       torch.tensor(KAT["unpack_int4"]["codes"], dtype=torch.int8))


def test_pack_unpack_round_trip():
    torch.manual_seed(0)
    q = torch.randint(-7, 8, (4, 128), dtype=torch.int8)
    assert torch.equal(unpack_int4(pack_int4(q)), q)


def test_quantize_known_values():
    k = KAT["quantize_groupwise"]
    q, s = quantize_groupwise(t16(k["weights_f16"]), group_size=k["group_size"])
    assert torch.equal(q, torch.tensor(k["codes"], dtype=torch.int8))
    assert torch.equal(s, t16(k["scales_f16"]))
    k = KAT["quantize_and_pack"]
    p, s = quantize_and_pack_weights(t16(k["weights_f16"]), group_size=k["group_size"])
    assert torch.equal(p, torch.tensor(k["packed"], dtype=torch.uint8))
    assert torch.equal(s, t16(k["scales_f16"]))


@pytest.mark.parametrize("call,exc", [
    (lambda: pack_int4(torch.zeros((1, 4), dtype=torch.int16)), TypeError),
    (lambda: pack_int4(torch.zeros((4,), dtype=torch.int8)), ValueError),
    (lambda: pack_int4(torch.zeros((1, 3), dtype=torch.int8)), ValueError),
    (lambda: pack_int4(torch.full((1, 2), 8, dtype=torch.int8)), ValueError),
    (lambda: unpack_int4(torch.zeros((1, 4), dtype=torch.int8)), TypeError),
    (lambda: quantize_groupwise(torch.zeros((2, 8), dtype=torch.float64)), TypeError),
    (lambda: quantize_groupwise(torch.zeros((2, 8)), group_size=0), ValueError),
    (lambda: quantize_groupwise(torch.zeros((2, 12)), group_size=8), ValueError),
])
def test_quantization_errors(call, exc):
    with pytest.raises(exc):
        call()


def test_quantizer_matches_oracle_bytes():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((96, 1024)) * 0.02).astype(np.float32)
    w[5, :128] = 0
    p, s = quantize_and_pack_weights(torch.from_numpy(w), 128)
    po, so = oracle.quantize_and_pack(w, 128)
    assert np.array_equal(p.numpy(), po)
    assert np.array_equal(s.numpy().view(np.uint16), so.view(np.uint16))


# ---------------------------------------------------------- reference ----
def test_dequantize_known_values():
    k = KAT["dequantize"]
    p = pack_int4(torch.tensor(k["codes"], dtype=torch.int8))
    w = dequantize_weights(p, t16(k["scales_f16"]), group_size=k["group_size"])
    assert torch.equal(w, torch.tensor(k["weights_f32"], dtype=torch.float32))


def test_linear_reference_known_values():
    k = KAT["linear"]
    p = pack_int4(torch.tensor(k["codes"], dtype=torch.int8))
    out = linear_reference(t16(k["activations_f16"]), p, t16(k["scales_f16"]), group_size=k["group_size"])
    assert torch.equal(out, t16(k["output_f16"]))


def test_cpu_path_matches_oracle():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 512)).astype(np.float16)
    packed = rng.integers(0, 256, (40, 256), dtype=np.uint8)
    scales = (rng.random((40, 4)) + 0.01).astype(np.float16)
    got = linear_reference(torch.from_numpy(x), torch.from_numpy(packed), torch.from_numpy(scales), 128)
    ref = oracle.linear(x, packed, scales, 128).astype(np.float32)
    assert np.all(np.abs(got.float().numpy() - ref) <= 1e-2 * (1 + np.abs(ref)))
    deq = dequantize_weights(torch.from_numpy(packed), torch.from_numpy(scales), 128).to(torch.float16)
    assert np.array_equal(deq.numpy().view(np.uint16), oracle.dequantize_f16(packed, scales, 128).view(np.uint16))


# --------------------------------------------------------- checkpoint ----
def test_checkpoint_round_trip(tmp_path):
    p, s = quantize_and_pack_weights(t16([[0.25, -0.375, 0.875, -0.125]]), group_size=4)
    path = tmp_path / "q.pt"
    save_quantized_weight_checkpoint(path, p, s, group_size=4)
    lp, ls, g = load_quantized_weight_checkpoint(path)
    assert torch.equal(lp, p) and torch.equal(ls, s) and g == 4
    raw = torch.load(path, weights_only=True)
    assert raw["format"] == "w4a16-linear" and raw["version"] == 1 and tuple(raw["original_shape"]) == (1, 4)


def test_checkpoint_rejects_bad_format(tmp_path):
    p, s = quantize_and_pack_weights(t16([[0.25, -0.375, 0.875, -0.125]]), group_size=4)
    path = tmp_path / "q.pt"
    torch.save({"format": "other", "version": 1, "packed_weights": p, "scales": s, "group_size": 4,
                "original_shape": (1, 4)}, path)
    with pytest.raises(ValueError, match="unsupported format"):
        load_quantized_weight_checkpoint(path)
    torch.save({"format": "w4a16-linear", "version": 2, "packed_weights": p, "scales": s, "group_size": 4,
                "original_shape": (1, 4)}, path)
    with pytest.raises(ValueError, match="unsupported version"):
        load_quantized_weight_checkpoint(path)


# ------------------------------------------------------------- module ----
def _kat_layer(**kw):
    k = KAT["module"]
    p, s = quantize_and_pack_weights(t16(k["weights_f16"]), group_size=k["group_size"])
    return QuantizedLinear(p, s, group_size=k["group_size"], **kw)


def test_module_known_values():
    layer = _kat_layer()
    out = layer(t16(KAT["module"]["activations_f16"]))
    assert torch.equal(out, t16(KAT["module"]["output_f16"]))
    assert "packed_weights" in layer.state_dict() and "scales" in layer.state_dict()


def test_module_empty_shapes():
    layer = QuantizedLinear.empty(out_features=2, in_features=4, group_size=4, bias=True, fused=False)
    assert layer.packed_weights.shape == (2, 2) and layer.packed_weights.dtype == torch.uint8
    assert layer.scales.shape == (2, 1) and layer.scales.dtype == torch.float16
    assert layer.bias is not None and layer.bias.shape == (2,) and layer.fused is False
    with pytest.raises(ValueError, match="K must be divisible by group_size"):
        QuantizedLinear.empty(out_features=2, in_features=6, group_size=4)


def test_module_from_float_exact():
    k = KAT["module"]
    lin = torch.nn.Linear(4, 2, bias=True, dtype=torch.float16)
    with torch.no_grad():
        lin.weight.copy_(t16(k["weights_f16"]))
        lin.bias.copy_(t16(k["bias_f16"]))
    q = QuantizedLinear.from_float(lin, group_size=4)
    x = t16(k["activations_f16"][0])
    assert torch.equal(q(x), lin(x))
    assert torch.equal(q.bias, lin.bias)


def test_module_errors():
    layer = _kat_layer()
    with pytest.raises(TypeError, match="activations must have dtype torch.float16"):
        layer(torch.ones((2, 4)))
    with pytest.raises(RuntimeError, match="activations must not require grad"):
        layer(torch.ones((2, 4), dtype=torch.float16, requires_grad=True))
    with pytest.raises(ValueError):
        layer(torch.ones((2, 6), dtype=torch.float16))
    with pytest.raises(TypeError):
        QuantizedLinear.from_float(torch.nn.Conv1d(1, 1, 1))
    with pytest.raises(ValueError):
        QuantizedLinear(torch.zeros((2, 2), dtype=torch.uint8), torch.zeros((2, 2), dtype=torch.float16), 4)


# -------------------------------------------------------- integration ----
class Toy(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.direct = torch.nn.Linear(4, 2, bias=True, dtype=torch.float16)
        self.nested = torch.nn.Sequential(torch.nn.Linear(4, 2, bias=False, dtype=torch.float16))
        w = t16(KAT["module"]["weights_f16"])
        with torch.no_grad():
            self.direct.weight.copy_(w)
            self.direct.bias.copy_(t16(KAT["module"]["bias_f16"]))
            self.nested[0].weight.copy_(w)

    def forward(self, x):
        return self.direct(x) + self.nested(x)


class Shapes(torch.nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.direct = torch.nn.Linear(4, 2, bias=True, dtype=torch.float16)
        self.nested = torch.nn.Sequential(torch.nn.Linear(4, 2, bias=False, dtype=torch.float16))

    def forward(self, x):
        return self.direct(x) + self.nested(x)


X = t16(KAT["module"]["activations_f16"][0])


def test_replace_linear_layers():
    model = Toy()
    expected = model(X)
    assert replace_linear_layers(model, group_size=4) == 2
    assert isinstance(model.direct, QuantizedLinear) and isinstance(model.nested[0], QuantizedLinear)
    assert torch.equal(model(X), expected)


def test_replace_warns_on_unaligned():
    class Mixed(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.aligned = torch.nn.Linear(4, 2, dtype=torch.float16)
            self.nested = torch.nn.Sequential(torch.nn.Linear(6, 2, bias=False, dtype=torch.float16))

    model = Mixed()
    with pytest.warns(UserWarning, match=r"nested\.0"):
        assert replace_linear_layers(model, group_size=4) == 1
    assert isinstance(model.nested[0], torch.nn.Linear)


def test_replace_fused_flag_and_packed_only_round_trip():
    model = Toy()
    assert replace_linear_layers(model, group_size=4, fused=False) == 2
    assert model.direct.fused is False and model.nested[0].fused is False
    expected = model(X)
    state = {k: v.clone() for k, v in model.state_dict().items()}
    target = Toy()
    with torch.no_grad():
        target.direct.weight.fill_(3.0)
    assert replace_linear_layers(target, group_size=4, packed_only=True) == 2
    target.load_state_dict(state)
    assert torch.equal(target(X), expected)


def test_load_packed_state_dict_from_meta():
    source = Toy()
    replace_linear_layers(source, group_size=4, fused=False)
    expected = source(X)
    state = {k: v.clone() for k, v in source.state_dict().items()}
    with torch.device("meta"):
        target = Shapes()
    assert load_packed_state_dict(target, state, group_size=4, device="cpu", fused=False) == 2
    assert target.direct.packed_weights.device.type == "cpu"
    assert "weight" not in target.direct.state_dict()
    assert torch.equal(target(X), expected)


def test_tiny_hf_llama_round_trip():
    transformers = pytest.importorskip("transformers")
    config = transformers.LlamaConfig(vocab_size=32, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=32,
                                      rms_norm_eps=1e-5, tie_word_embeddings=False)
    torch.manual_seed(0)
    try:
        source = transformers.AutoModelForCausalLM.from_config(config, dtype=torch.float16)
    except TypeError:
        source = transformers.AutoModelForCausalLM.from_config(config, torch_dtype=torch.float16)
    source.eval()
    replace_linear_layers(source, group_size=64, fused=False)
    state = {k: v.detach().cpu().clone() for k, v in source.state_dict().items()}
    ids = torch.randint(0, 32, (1, 4))
    with torch.device("meta"):
        try:
            target = transformers.AutoModelForCausalLM.from_config(config, dtype=torch.float16)
        except TypeError:
            target = transformers.AutoModelForCausalLM.from_config(config, torch_dtype=torch.float16)
    assert load_packed_state_dict(target, state, group_size=64, device="cpu", fused=False) > 0
    target.eval()
    with torch.inference_mode():
        expected = source(input_ids=ids).logits
        result = target(input_ids=ids).logits
    assert not any(isinstance(m, torch.nn.Linear) for m in target.modules() if m is not target)
    assert torch.equal(source.model.rotary_emb.inv_freq, target.model.rotary_emb.inv_freq)
    assert torch.equal(result, expected)
