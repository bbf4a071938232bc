"""GPU tests of the drop-in API: the torch ops and QuantizedLinear on the HIP
kernels (the reference's tests/test_cuda.py and the GPU half of
tests/test_linear.py / tests/test_integration.py), HIP-graph replay safety,
and the Llama decode model. Parity bar against the CPU oracle: |err| <=
1e-2 (1 + |ref|); dequantize bit-identical."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
import w4a16
from w4a16.cuda import dequantize_cuda, linear_cuda
from w4a16.linear import QuantizedLinear
from w4a16.quantization import quantize_and_pack_weights
from nibble_amd import _lib
from tests._cases import assert_parity, expected, make_case

pytestmark = pytest.mark.gpu


def _on(dev, *ts):
    return [t.to(dev) for t in ts]


@pytest.mark.parametrize("m,k,n", [(4, 256, 8), (1, 256, 8), (1, 2048, 2048), (1, 2048, 5632), (1, 5632, 2048),
                                   (1, 256, 7), (9, 256, 8), (3, 2048, 2048), (8, 256, 7), (6, 20480, 8200)])
def test_op_matches_oracle(gpu, m, k, n):
    """The torch op against the oracle; (6, 20480, 8200) takes the split-K
    kernel with a workspace from the caching allocator."""
    x, p, s = make_case(m, k, n, seed=m * 7 + k)
    out = linear_cuda(*_on(gpu, x, p, s), 128)
    assert out.dtype == torch.float16 and out.shape == (m, n)
    assert_parity(out, expected(x, p, s), f"op M={m} K={k} N={n}")


@pytest.mark.parametrize("decode", ["auto", "valu", "oneshot", "mfma"])
@pytest.mark.parametrize("rows_per_warp", ["1", "2", "4"])
def test_env_selected_kernels(gpu, monkeypatch, decode, rows_per_warp):
    monkeypatch.setenv("W4A16_DECODE", decode)
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", rows_per_warp)
    for m in (1, 3):
        x, p, s = make_case(m, 2048, 200, seed=11)
        assert_parity(linear_cuda(*_on(gpu, x, p, s), 128), expected(x, p, s), f"{decode}/{rows_per_warp} M={m}")


def test_op_rejects_bad_rows_per_warp(gpu, monkeypatch):
    x, p, s = make_case(1, 256, 8)
    monkeypatch.setenv("W4A16_ROWS_PER_WARP", "3")
    with pytest.raises(RuntimeError):
        linear_cuda(*_on(gpu, x, p, s), 128)


def test_op_rejects(gpu):
    x, p, s = make_case(4, 256, 8)
    xd, pd, sd = _on(gpu, x, p, s)
    with pytest.raises(RuntimeError):
        linear_cuda(xd.float(), pd, sd, 128)                               # fp32 activations
    wide = torch.randn((4, 512), dtype=torch.float16, device=gpu)[:, :256]
    with pytest.raises(RuntimeError):
        linear_cuda(wide, pd, sd, 128)                                     # non-contiguous
    with pytest.raises(RuntimeError):
        linear_cuda(xd[:, :128].contiguous(), pd, sd, 128)                  # K mismatch
    with pytest.raises(RuntimeError):
        linear_cuda(x, p, s, 128)                                          # CPU tensors
    _, p48, s48 = make_case(1, 96, 8, group_size=48)
    with pytest.raises(RuntimeError):
        dequantize_cuda(*_on(gpu, p48, s48), 48)                          # dequantize needs G % 32 == 0


def test_misaligned_activations(gpu):
    x, p, s = make_case(1, 2048, 64, seed=9)
    buf = torch.empty(2049, dtype=torch.float16, device=gpu)
    buf[1:] = x.to(gpu)[0]
    xd = buf[1:].view(1, 2048)
    assert xd.data_ptr() % 16 != 0 and xd.is_contiguous()
    assert_parity(linear_cuda(xd, *_on(gpu, p, s), 128), expected(x, p, s), "misaligned")


@pytest.mark.parametrize("g", [32, 64, 128])
def test_dequantize_op_bit_identical(gpu, g):
    _, p, s = make_case(1, 2048, 300, seed=g, group_size=g)
    w = dequantize_cuda(*_on(gpu, p, s), g)
    assert w.dtype == torch.float16 and w.shape == (300, 2048)
    assert np.array_equal(w.cpu().numpy().view(np.uint16), oracle.dequantize_f16(p.numpy(), s.numpy(), g).view(np.uint16))


# --------------------------------------------------------- module (GPU) ----
def test_module_bias_small_batch(gpu):
    x, p, s = make_case(2, 128, 8, seed=1)
    bias = torch.randn((8,), dtype=torch.float16)
    layer = QuantizedLinear(*_on(gpu, p, s), group_size=128, bias=bias.to(gpu))
    out = layer(x.to(gpu))
    ref = torch.from_numpy(expected(x, p, s)) + bias.float()
    assert_parity(out, ref.numpy(), "bias")


def test_module_noncontiguous_and_3d(gpu):
    x, p, s = make_case(6, 256, 16, seed=2)
    layer = QuantizedLinear(*_on(gpu, p, s), group_size=128)
    wide = torch.zeros((6, 512), dtype=torch.float16)
    wide[:, :256] = x
    view = wide.to(gpu)[:, :256]
    assert not view.is_contiguous()
    assert_parity(layer(view), expected(x, p, s), "non-contiguous")
    out3 = layer(x.to(gpu).view(2, 3, 256))
    assert out3.shape == (2, 3, 16)
    assert_parity(out3.reshape(6, 16), expected(x, p, s), "3-D")


@pytest.mark.parametrize("fused,m,k,n", [(True, 16, 128, 8), (True, 300, 128, 8), (True, 600, 128, 8), (False, 1, 128, 8),
                                         (False, 4, 128, 8), (True, 64, 2048, 5632), (True, 256, 4096, 512),
                                         (True, 9, 5632, 300)])
def test_module_prefill_paths_match_dequant_linear(gpu, fused, m, k, n):
    """Prompts: fused layers run the W4A16 GEMM up to NATIVE_GEMM_MAX_ROWS
    rows, longer prompts and fused=False layers dequantize + F.linear
    (hipBLASLt); every path agrees with F.linear on the dequantized fp16
    weights at the reference's prefill tolerance (reference
    tests/test_linear.py:207-243, rtol = atol = 1e-3)."""
    from nibble_amd.linear import NATIVE_GEMM_MAX_ROWS

    x, p, s = make_case(m, k, n, seed=3 + m)
    layer = QuantizedLinear(*_on(gpu, p, s), group_size=128, fused=fused)
    w16 = torch.from_numpy(oracle.dequantize_f16(p.numpy(), s.numpy(), 128)).to(gpu)
    out = layer(x.to(gpu))
    torch.testing.assert_close(out, F.linear(x.to(gpu), w16), rtol=1e-3, atol=1e-3)
    if fused and 8 < m <= NATIVE_GEMM_MAX_ROWS:
        # the module's prompt rows are the op's, bit for bit
        assert torch.equal(out, linear_cuda(x.to(gpu), *_on(gpu, p, s), 128))


@pytest.mark.parametrize("m,k,n", [(16, 2048, 8192), (12, 2048, 32000), (9, 2048, 11264), (16, 5632, 2048),
                                   (13, 4096, 14336), (64, 2048, 5632)])
def test_module_prompt_rows_randn_weights(gpu, m, k, n):
    """Prompt rows of a fused layer with randn (not 0.02-scaled) weights, as
    reference tests/test_linear.py:207-225 makes them: every kernel the op
    routes 9..512 rows to must agree with F.linear on the dequantized fp16
    weights at rtol = atol = 1e-3 (the offset-decode kernels, whose sums run at
    ~1032 |x| per group, would not at these scales)."""
    torch.manual_seed(m + k + n)
    x = torch.randn((m, k), dtype=torch.float16, device=gpu)
    w = torch.randn((n, k), dtype=torch.float16, device=gpu)
    packed, scales = quantize_and_pack_weights(w, group_size=128)
    layer = QuantizedLinear(packed, scales, group_size=128, fused=True)
    print(f"[case] module prompt M={m} K={k} N={n} plan={_lib.plan_linear(x.data_ptr(), packed.data_ptr(), m, n, k)}",
          flush=True)
    torch.testing.assert_close(layer(x), F.linear(x, dequantize_cuda(packed, scales, 128)), rtol=1e-3, atol=1e-3)


def test_module_prefill_matches_dequant_linear_reference_case(gpu):
    """Reference tests/test_linear.py:207-225 with its inputs: fp16 randn
    weights quantized on the device, M = 16 > FUSED_MAX_ROWS."""
    torch.manual_seed(0)
    activations = torch.randn((16, 128), dtype=torch.float16, device=gpu)
    weights = torch.randn((8, 128), dtype=torch.float16, device=gpu)
    packed, scales = quantize_and_pack_weights(weights, group_size=128)
    layer = QuantizedLinear(packed, scales, group_size=128, fused=True)
    w16 = dequantize_cuda(packed, scales, 128)
    torch.testing.assert_close(layer(activations), F.linear(activations, w16), rtol=1e-3, atol=1e-3)


def test_module_prefill_odd_group_uses_generic_kernel(gpu):
    x, p, s = make_case(12, 96, 8, seed=4, group_size=48)
    layer = QuantizedLinear(*_on(gpu, p, s), group_size=48)
    assert_parity(layer(x.to(gpu)), expected(x, p, s, 48), "G=48 prefill")


def test_module_from_float_on_gpu_matches_oracle(gpu):
    torch.manual_seed(0)
    lin = torch.nn.Linear(2048, 512, bias=False, dtype=torch.float16, device=gpu)
    q = QuantizedLinear.from_float(lin, group_size=128)
    x = torch.randn((1, 2048), dtype=torch.float16)
    ref = oracle.linear(x.numpy(), q.packed_weights.cpu().numpy(), q.scales.cpu().numpy(), 128).astype(np.float32)
    assert_parity(q(x.to(gpu)), ref, "from_float")


def test_load_packed_state_dict_does_not_materialize_fp16(gpu):
    k, n = 2048, 2048
    src = QuantizedLinear.from_float(torch.nn.Linear(k, n, bias=False, dtype=torch.float16), group_size=128)
    state = {"layer.packed_weights": src.packed_weights.clone(), "layer.scales": src.scales.clone()}

    class Wrapper(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layer = torch.nn.Linear(k, n, bias=False, dtype=torch.float16)

    with torch.device("meta"):
        model = Wrapper()
    torch.cuda.empty_cache()
    before = torch.cuda.memory_allocated()
    assert w4a16.load_packed_state_dict(model, state, group_size=128, device="cuda") == 1
    delta = torch.cuda.memory_allocated() - before
    assert src.packed_weights.numel() + src.scales.numel() * 2 <= delta < k * n * 2


@pytest.mark.parametrize("rows", [1, 4, 24])
def test_traces_under_torch_compile(gpu, rows):
    torch.manual_seed(0)
    p, s = quantize_and_pack_weights(torch.randn((256, 512), dtype=torch.float16, device=gpu), 128)
    layer = QuantizedLinear(p, s, group_size=128)
    x = torch.randn((rows, 512), dtype=torch.float16, device=gpu)
    torch._dynamo.reset()
    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    with torch.inference_mode():
        torch.testing.assert_close(compiled(x), layer(x), rtol=1e-3, atol=1e-3)


# ----------------------------------------------------------- HIP graphs ----
def test_graph_replays_match_eager(gpu):
    """Ops captured in a HIP graph, replayed several times with eager work
    and synchronisations in between; every replay equals the eager result
    (the split-K case, whose workspace comes from the graph's pool, too)."""
    cases = [make_case(m, k, n, seed=m + n)
             for m, k, n in [(1, 2048, 512), (4, 2048, 512), (1, 5632, 300), (4, 20480, 8192)]]
    dev_cases = [_on(gpu, *c) for c in cases]
    eager = [linear_cuda(x, p, s, 128).clone() for x, p, s in dev_cases]
    deq_eager = dequantize_cuda(dev_cases[0][1], dev_cases[0][2], 128).clone()
    g = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            outs = [linear_cuda(x, p, s, 128) for x, p, s in dev_cases]
            deq = dequantize_cuda(dev_cases[0][1], dev_cases[0][2], 128)
    torch.cuda.current_stream().wait_stream(stream)
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        deq.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"
        assert torch.equal(deq, deq_eager)
        _ = torch.randn(1000, device=gpu).sum().item()   # unrelated eager work between replays


# ------------------------------------------------------------- decode -----
def test_llama_decode_graph_matches_eager(gpu):
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=8,
                      num_kv_heads=2, head_dim=32, max_seq_len=32)
    model = LlamaDecoder(cfg, device=gpu, seed=0)
    prompt = torch.randint(0, cfg.vocab_size, (12,), generator=torch.Generator().manual_seed(1)).to(gpu)
    eager = model.generate(prompt, 8, use_graph=False)
    model.prefill(prompt)
    model.capture()
    graphed = model.generate(prompt, 8, use_graph=True)
    assert torch.equal(eager, graphed)
    again = model.generate(prompt, 8, use_graph=True)
    assert torch.equal(eager, again)


def test_llama_full_size_builds_and_decodes(gpu):
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(max_seq_len=24)
    model = LlamaDecoder(cfg, device=gpu, seed=0)
    assert len(model.linear_layers()) == 155
    assert model.packed_bytes() == 533372928
    prompt = torch.randint(0, cfg.vocab_size, (16,), generator=torch.Generator().manual_seed(0)).to(gpu)
    model.prefill(prompt)
    model.capture()
    toks = model.generate(prompt, 4, use_graph=True)
    assert toks.shape == (4,) and int(toks.min()) >= 0 and int(toks.max()) < cfg.vocab_size
