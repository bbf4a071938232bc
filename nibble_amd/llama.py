"""A random-init Llama-architecture decoder whose linear layers are
``QuantizedLinear`` -- the caller that the end-to-end decode measurement
(tokens/s) exercises.

The reference measures decode on HuggingFace TinyLlama-1.1B with a static KV
cache and CUDA graphs (reference ``scripts/generate.py:260-365``); checkpoints
cannot be fetched here, so this module builds the same architecture offline:
22 layers, hidden 2048, intermediate 5632, 32 query / 4 key-value heads of
dim 64, vocab 32000, RMSNorm, rotary position embedding, SiLU-gated MLP.
All 155 linear layers (q, k, v, o, gate, up, down per layer, and lm_head)
hold INT4 group-128 weights quantized from N(0, 0.02).

Decode (one token, M = 1) runs the fused step of ``include/w4a16_decode.h``
by default: per layer, (1) RMSNorm + q|k|v GEMV over the concatenated
projection, (2) rotary embedding + KV-cache append + attention, (3) o GEMV +
residual, (4) RMSNorm + gate|up GEMV with the SiLU-multiply epilogue, (5)
down GEMV + residual; then RMSNorm + lm_head GEMV and the greedy argmax,
which also advances the position and gathers the next token's embedding: 5
launches per layer plus 2. While the position
is below 64 (and the head layout allows it), the rotary embedding and the
KV-cache append move into the q|k|v GEMV's epilogue
(``w4a16_gemv_qkv_rope_f16``) and attention + o GEMV + residual are one
launch (``w4a16_attention_o_cached_f16``: every o-projection workgroup
recomputes the one-chunk attention on the matrix cores), so a step is 4
launches per layer; the host tracks the position to pick that step
(``qkv_rope=False`` keeps rotary and append in the attention launch,
``w4a16_attention_o_f16``). The q/k/v and
gate/up weights live in one buffer each, and every ``QuantizedLinear`` keeps
a contiguous view of its rows, so state-dict keys and layouts are those of
the per-layer modules. ``fused=False`` runs the same step as separate torch
ops around ``QuantizedLinear`` (the reference-shaped decoder).

Prefill of a prompt runs the W4A16 op itself for every projection up to 1024
tokens (q|k|v as one op; the op's W4A16 GEMM from 9 rows, its LDS-staged
form from 128; up to 8 rows its small-batch kernels), gate|up as one GEMM
with the SiLU-multiply in its epilogue, and one launch each for the residual
add + RMSNorm and the rotary + KV append + causal attention; from 1025 tokens
the projections take dequantize + hipBLASLt. The attention launch holds up
to 256 cache slots in LDS and streams longer prompts through it in 256-slot
blocks where query heads per KV head are a power of two up to 64; other
head layouts run prompts past 256 tokens as torch ops around the same op. ``capture_prefill(T)`` records
a T-token prefill in a HIP graph. ``Decoder.capture()`` records one decode step -- embedding, 22 blocks,
lm_head, greedy argmax, KV-cache write and position increment -- in a HIP
graph, so generating a token is one ``graph.replay()``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from nibble_amd import _lib
from nibble_amd.cuda import dequantize_cuda
from nibble_amd.linear import QuantizedLinear
from nibble_amd.quantization import quantize_and_pack_weights

# Longest prompt the fused prefill takes where the prefill attention cannot
# stream the caches (query heads per KV head not a power of two up to 64:
# w4a16_prefill_attention_f16 then holds at most 256 cache slots in LDS);
# elsewhere it takes any prompt that fits the cache.
FUSED_PREFILL_MAX_TOKENS = 256
# Most rows a prefill projection sends to the W4A16 op in the torch-op
# prefill; more rows take dequantize + hipBLASLt. Measured on the 1.1B and 8B
# layer shapes: the op's GEMM is 1.2-3x faster than dequantize + hipBLASLt
# from 32 to 256 rows, except 4096 x 14336 at 256 rows (90.7 against 80.7 us).
NATIVE_PREFILL_MAX_ROWS = 256
# Most rows a fused-prefill projection sends to the W4A16 op (the GEMM and its
# SiLU form); longer prompts take dequantize + hipBLASLt. Measured on the whole
# 1.1B prefill (one HIP graph): 1024 tokens 4.31 ms with the op against 4.88
# with dequantize + hipBLASLt from 513 rows; 2048 tokens 7.65 against 7.53.
FUSED_PREFILL_NATIVE_MAX_ROWS = 1024


@dataclass
class LlamaConfig:
    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_layers: int = 22
    num_heads: int = 32
    num_kv_heads: int = 4
    head_dim: int = 64
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_seq_len: int = 64
    group_size: int = 128
    init_std: float = 0.02

    @property
    def num_linear_layers(self) -> int:
        return self.num_layers * 7 + 1


def _quantized(out_features: int, in_features: int, cfg: LlamaConfig, device, gen) -> QuantizedLinear:
    """Random N(0, init_std) weights quantized RTN to INT4, or (gen is None)
    uninitialised packed storage for a later load_state_dict."""
    if gen is None:
        return QuantizedLinear.empty(out_features, in_features, group_size=cfg.group_size, device=device)
    weight = torch.randn((out_features, in_features), device=device, generator=gen) * cfg.init_std
    packed, scales = quantize_and_pack_weights(weight, cfg.group_size)
    return QuantizedLinear(packed, scales, group_size=cfg.group_size)


class RMSNorm(torch.nn.Module):
    def __init__(self, dim: int, eps: float, device) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(dim, dtype=torch.float16, device=device), requires_grad=False)
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return (xf * self.weight.float()).to(torch.float16)


class Block(torch.nn.Module):
    def __init__(self, cfg: LlamaConfig, device, gen) -> None:
        super().__init__()
        h, kv = cfg.hidden_size, cfg.num_kv_heads * cfg.head_dim
        self.cfg = cfg
        self.input_norm = RMSNorm(h, cfg.rms_norm_eps, device)
        self.q_proj = _quantized(h, h, cfg, device, gen)
        self.k_proj = _quantized(kv, h, cfg, device, gen)
        self.v_proj = _quantized(kv, h, cfg, device, gen)
        self.o_proj = _quantized(h, h, cfg, device, gen)
        self.post_norm = RMSNorm(h, cfg.rms_norm_eps, device)
        self.gate_proj = _quantized(cfg.intermediate_size, h, cfg, device, gen)
        self.up_proj = _quantized(cfg.intermediate_size, h, cfg, device, gen)
        self.down_proj = _quantized(h, cfg.intermediate_size, cfg, device, gen)
        # concatenated q|k|v and gate|up storage (set by LlamaDecoder)
        self.qkv_packed = self.qkv_scales = self.gu_packed = self.gu_scales = None
        self.native_prefill = True

    def _native(self, x: torch.Tensor, packed: torch.Tensor) -> bool:
        """Whether the W4A16 op itself (not dequantize + hipBLASLt) is the fast
        path for these rows: GPU rows (at most NATIVE_PREFILL_MAX_ROWS) that
        the op routes to a tuned kernel or its GEMM."""
        if not (self.native_prefill and x.is_cuda and x.shape[0] <= NATIVE_PREFILL_MAX_ROWS):
            return False
        plan = _lib.plan_linear(x.data_ptr(), packed.data_ptr(), x.shape[0], packed.shape[0], x.shape[1],
                                self.cfg.group_size)
        return plan["kernel"] != "generic"

    def _linear(self, mod: QuantizedLinear, x: torch.Tensor) -> torch.Tensor:
        if self._native(x, mod.packed_weights):
            return torch.ops.w4a16.linear(x, mod.packed_weights, mod.scales, self.cfg.group_size)
        return mod(x)

    def forward(self, x, cos, sin, positions, k_cache, v_cache, mask):
        """x [T, H] fp16; positions [T] int64 (cache slots to write);
        k_cache / v_cache [kv_heads, S, head_dim]; mask [T, S] additive fp32.
        With native_prefill on a GPU, prompts of up to NATIVE_PREFILL_MAX_ROWS
        tokens run q|k|v and gate|up as one W4A16 op each over the
        concatenated weights (and o, down as the op); otherwise every
        projection is its QuantizedLinear."""
        cfg = self.cfg
        t = x.shape[0]
        kv = cfg.num_kv_heads * cfg.head_dim
        h = self.input_norm(x)
        if self.qkv_packed is not None and self._native(h, self.qkv_packed):
            qkv = torch.ops.w4a16.linear(h, self.qkv_packed, self.qkv_scales, cfg.group_size)
            q = qkv[:, : cfg.hidden_size].reshape(t, cfg.num_heads, cfg.head_dim)
            k = qkv[:, cfg.hidden_size: cfg.hidden_size + kv].reshape(t, cfg.num_kv_heads, cfg.head_dim)
            v = qkv[:, cfg.hidden_size + kv:].reshape(t, cfg.num_kv_heads, cfg.head_dim)
        else:
            q = self.q_proj(h).view(t, cfg.num_heads, cfg.head_dim)
            k = self.k_proj(h).view(t, cfg.num_kv_heads, cfg.head_dim)
            v = self.v_proj(h).view(t, cfg.num_kv_heads, cfg.head_dim)
        q = _rope(q, cos, sin)
        k = _rope(k, cos, sin)
        k_cache.index_copy_(1, positions, k.transpose(0, 1).contiguous())
        v_cache.index_copy_(1, positions, v.transpose(0, 1).contiguous())
        group = cfg.num_heads // cfg.num_kv_heads
        # attention in fp32 on contiguous operands
        kf = k_cache.float().repeat_interleave(group, dim=0)            # [heads, S, d]
        vf = v_cache.float().repeat_interleave(group, dim=0)
        qf = q.float().transpose(0, 1).contiguous()                     # [heads, T, d]
        scores = torch.matmul(qf, kf.transpose(1, 2).contiguous()) / math.sqrt(cfg.head_dim) + mask
        attn = torch.matmul(torch.softmax(scores, dim=-1), vf)          # [heads, T, d]
        attn = attn.transpose(0, 1).reshape(t, cfg.hidden_size).to(torch.float16)
        x = x + self._linear(self.o_proj, attn)
        h = self.post_norm(x)
        if self.gu_packed is not None and self._native(h, self.gu_packed):
            gu = torch.ops.w4a16.linear(h, self.gu_packed, self.gu_scales, cfg.group_size)
            mlp = F.silu(gu[:, : cfg.intermediate_size]) * gu[:, cfg.intermediate_size:]
        else:
            mlp = F.silu(self.gate_proj(h)) * self.up_proj(h)
        x = x + self._linear(self.down_proj, mlp)
        return x


def _concat_rows(modules: list[QuantizedLinear]) -> tuple[torch.Tensor, torch.Tensor]:
    """Move the modules' packed weights and scales into one buffer each (rows
    stacked in order) and point every module at a contiguous view of its rows."""
    packed = torch.cat([m.packed_weights for m in modules])
    scales = torch.cat([m.scales for m in modules])
    row = 0
    for m in modules:
        n = m.out_features
        m.packed_weights = packed[row: row + n]
        m.scales = scales[row: row + n]
        row += n
    return packed, scales


def _rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotary embedding, half-split convention; x [T, heads, d], cos/sin [T, d/2]."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half].float(), x[..., half:].float()
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(x.dtype)


class LlamaDecoder(torch.nn.Module):
    """Random-init Llama with INT4 linear layers, a static KV cache and greedy decode."""

    def __init__(self, cfg: LlamaConfig, device: str | torch.device = "cuda", seed: int = 0,
                 fused: bool = True, init: str = "random", fuse_attention_o: bool = True) -> None:
        """init="random": N(0, init_std) weights (seeded); init="empty":
        uninitialised storage for load_state_dict (e.g. from
        nibble_amd.model_checkpoint.decoder_from_checkpoint).
        fuse_attention_o=False keeps attention and the o GEMV as two launches
        at every position."""
        super().__init__()
        if init not in ("random", "empty"):
            raise ValueError("init must be 'random' or 'empty'")
        self.cfg = cfg
        device = torch.device(device)
        # The fused step is HIP-only (CPU runs the torch ops) and built for
        # head_dim 64 and rows of K <= 16384.
        self.fused = (fused and device.type == "cuda" and cfg.head_dim == 64
                      and max(cfg.hidden_size, cfg.intermediate_size) <= 16384)
        # attention + o projection as one launch (positions < 64): head layouts
        # the kernel supports
        self.attn_o = (self.fused and fuse_attention_o and cfg.num_kv_heads in (1, 2, 4, 8)
                       and cfg.num_heads % cfg.num_kv_heads == 0 and cfg.num_heads // cfg.num_kv_heads <= 16
                       and cfg.num_heads * cfg.head_dim <= 4096 and cfg.group_size == 128)
        gen = torch.Generator(device=device).manual_seed(seed) if init == "random" else None
        if gen is None:
            table = torch.empty((cfg.vocab_size, cfg.hidden_size), dtype=torch.float16, device=device)
        else:
            table = (torch.randn((cfg.vocab_size, cfg.hidden_size), device=device, generator=gen)
                     * cfg.init_std).to(torch.float16)
        self.embed = torch.nn.Parameter(table, requires_grad=False)
        self.layers = torch.nn.ModuleList([Block(cfg, device, gen) for _ in range(cfg.num_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device)
        self.lm_head = _quantized(cfg.vocab_size, cfg.hidden_size, cfg, device, gen)
        inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, device=device).float() / cfg.head_dim))
        angles = torch.outer(torch.arange(cfg.max_seq_len, device=device).float(), inv_freq)
        self.register_buffer("cos", angles.cos(), persistent=False)
        self.register_buffer("sin", angles.sin(), persistent=False)
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        shape = (cfg.num_layers, cfg.num_kv_heads, cfg.max_seq_len, cfg.head_dim)
        self.register_buffer("k_cache", torch.zeros(shape, dtype=torch.float16, device=device), persistent=False)
        self.register_buffer("v_cache", torch.zeros(shape, dtype=torch.float16, device=device), persistent=False)
        self.slots = torch.arange(cfg.max_seq_len, device=device)
        # static decode-step state (graph inputs/outputs)
        self.token = torch.zeros((1,), dtype=torch.int64, device=device)
        self.position = torch.zeros((1,), dtype=torch.int64, device=device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.graph_short: torch.cuda.CUDAGraph | None = None   # attention + o fused (position < 64)
        # several short steps in one graph (capture(tokens_per_replay=T)): graphs of T, T // 2, .. (> 1)
        # steps; step j's token goes to multi_tokens[j]. graph_multi is the T-step one.
        self.graph_multi: torch.cuda.CUDAGraph | None = None
        self.graphs_multi: dict[int, torch.cuda.CUDAGraph] = {}
        self.multi_tokens: torch.Tensor | None = None
        # position < 64: rotary + KV append in the q|k|v GEMV's epilogue (else in the attention + o launch)
        self.qkv_rope = True
        self.host_position = 0   # host copy of `position` (set by prefill, +1 per step)
        self.prefill_graph: torch.cuda.CUDAGraph | None = None
        self.fuse_prefill = True   # fused prefill (see fused_prefill)
        self.prefill_tokens: torch.Tensor | None = None
        self.prefill_positions: torch.Tensor | None = None
        # fused-step weights (views keep the per-module state-dict entries) and work buffers
        self.qkv = [_concat_rows([b.q_proj, b.k_proj, b.v_proj]) for b in self.layers]
        self.gate_up = [_concat_rows([b.gate_proj, b.up_proj]) for b in self.layers]
        for b, (qw, qs), (gw, gs) in zip(self.layers, self.qkv, self.gate_up):
            b.qkv_packed, b.qkv_scales, b.gu_packed, b.gu_scales = qw, qs, gw, gs
        h, kv = cfg.hidden_size, cfg.num_kv_heads * cfg.head_dim
        self.x_buf = torch.zeros((h,), dtype=torch.float16, device=device)
        self.qkv_buf = torch.zeros((h + 2 * kv,), dtype=torch.float16, device=device)
        self.attn_buf = torch.zeros((cfg.num_heads * cfg.head_dim,), dtype=torch.float16, device=device)
        # caches past 512 slots: the decode attention split into shares of the
        # slots (a workgroup per head and share, 256 workgroups where the heads
        # allow) and merged per head; 0 keeps one workgroup per head. 1.1B
        # model, graph-replayed decode: 2048 slots at position 1500 1837
        # against 1597 tok/s, 1024 at 900 1907 against 1830, 512 at 300 1970
        # against 2030 (so 512 slots keep the single launch); at most 64
        # shares, the split launch's limit
        self.attn_splits = (min(max(1, 256 // cfg.num_heads), max(1, cfg.max_seq_len // 128), 64)
                            if cfg.max_seq_len > 512 else 0)
        self.attn_ws = torch.empty((max(1, cfg.num_heads * self.attn_splits * 66),), dtype=torch.float32,
                                   device=device)
        self.mlp_buf = torch.zeros((cfg.intermediate_size,), dtype=torch.float16, device=device)
        self.logits = torch.zeros((cfg.vocab_size,), dtype=torch.float16, device=device)

    def linear_layers(self) -> list[QuantizedLinear]:
        return [m for m in self.modules() if isinstance(m, QuantizedLinear)]

    def packed_bytes(self) -> int:
        return sum(m.packed_weights.numel() + m.scales.numel() * 2 for m in self.linear_layers())

    def _forward(self, tokens: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """tokens [T], positions [T] -> logits of the last position [vocab] fp16."""
        x = self.embed[tokens]
        cos, sin = self.cos[positions], self.sin[positions]
        # additive mask: slot s visible to query t iff s <= positions[t]
        mask = torch.where(self.slots.unsqueeze(0) <= positions.unsqueeze(1), 0.0, float("-inf"))
        for i, layer in enumerate(self.layers):
            x = layer(x, cos, sin, positions, self.k_cache[i], self.v_cache[i], mask)
        return self.lm_head(self.norm(x[-1:]))[0]

    def fused_prefill(self, tokens: int) -> bool:
        """Whether a prompt of `tokens` tokens takes the fused prefill: the W4A16
        op for every projection and one launch for each RMSNorm, attention and
        SiLU-multiply (1 <= tokens <= max_seq_len; past FUSED_PREFILL_MAX_TOKENS
        only where the attention streams the caches through LDS, query heads
        per KV head a power of two up to 64)."""
        group = self.cfg.num_heads // self.cfg.num_kv_heads
        streams = group & (group - 1) == 0 and group <= 64
        limit = self.cfg.max_seq_len if streams else min(self.cfg.max_seq_len, FUSED_PREFILL_MAX_TOKENS)
        return self.fused and self.fuse_prefill and 1 <= tokens <= limit

    def _prefill(self, prompt: torch.Tensor, positions: torch.Tensor) -> None:
        if self.fused_prefill(prompt.numel()):
            # no cache reset: every fused attention kernel selects away the
            # slots past the position it attends to, whatever they hold
            self._prefill_fused(prompt)
            return
        self.k_cache.zero_()
        self.v_cache.zero_()
        logits = self._forward(prompt, positions)
        self.token.copy_(torch.argmax(logits).view(1))
        self.position.fill_(prompt.numel())
        if self.fused:
            _lib.embedding_f16(self.embed, self.token, self.x_buf)   # the first decode step's input

    def _prefill_fused(self, prompt: torch.Tensor) -> None:
        """The prompt (cache slots 0 .. T-1) with the decode step's roundings:
        RMSNorm of the embeddings, then per layer the q|k|v op, rotary + KV
        append + causal attention, the o op, residual add + RMSNorm
        (w4a16_prefill_attention_o_add_rmsnorm_f16: at 9..16 tokens the
        attention runs inside the o op's launch and the norm's launch sums
        its K slices), the gate|up projection with its SiLU * up epilogue,
        the down op with the residual add + the next RMSNorm (the next
        layer's input norm, or the final norm after the last layer;
        w4a16_linear_add_rmsnorm_f16 sums the op's K slices in the norm's
        launch); then the lm_head GEMV on the last normed row and the greedy
        argmax, which also gathers the first decode step's input row. 6
        launches per layer at 9..16 tokens, 7 otherwise. The embedding
        gather, the first RMSNorm and the position after the prompt are one
        launch (w4a16_embed_rmsnorm_f16)."""
        cfg = self.cfg
        t = prompt.numel()
        g = cfg.group_size
        first = self.layers[0].input_norm
        one_launch = cfg.hidden_size % 8 == 0 and cfg.hidden_size <= 8192 and self.embed.is_contiguous()
        if one_launch:
            # the embedding rows, their RMSNorm and the position after the prompt in one launch
            x = torch.empty((t, cfg.hidden_size), dtype=torch.float16, device=prompt.device)
            h = torch.empty_like(x)
            _lib.embed_rmsnorm_f16(self.embed, prompt.contiguous(), first.weight, first.eps, x, h,
                                   position=self.position)
        else:
            x = self.embed[prompt]
            h = torch.empty_like(x)
            _lib.rmsnorm_f16(x, first.weight, first.eps, h)
        attn = (torch.empty((t, cfg.num_heads * cfg.head_dim), dtype=torch.float16, device=x.device)
                if t > FUSED_PREFILL_NATIVE_MAX_ROWS else None)
        mlp = torch.empty((t, cfg.intermediate_size), dtype=torch.float16, device=x.device)
        for i, b in enumerate(self.layers):
            qkv_w, qkv_s = self.qkv[i]
            gu_w, gu_s = self.gate_up[i]
            qkv = self._prefill_linear(h, qkv_w, qkv_s)
            if t <= FUSED_PREFILL_NATIVE_MAX_ROWS:
                # attention + o + residual add + norm (9..16 tokens: the attention inside the o op's launch)
                _lib.prefill_attention_o_add_rmsnorm_f16(
                    qkv, self.k_cache[i], self.v_cache[i], self.cos, self.sin, 0, b.o_proj.packed_weights,
                    b.o_proj.scales, x, b.post_norm.weight, b.post_norm.eps, x, h, cfg.num_heads, cfg.num_kv_heads,
                    cfg.head_dim, g)
            else:
                _lib.prefill_attention_f16(qkv, self.k_cache[i], self.v_cache[i], self.cos, self.sin, 0, attn,
                                           cfg.num_heads, cfg.num_kv_heads, cfg.head_dim)
                o = self._prefill_linear(attn, b.o_proj.packed_weights, b.o_proj.scales)
                _lib.add_rmsnorm_f16(x, o, b.post_norm.weight, b.post_norm.eps, x, h)
            if t <= FUSED_PREFILL_NATIVE_MAX_ROWS:
                _lib.linear_silu_f16(h, gu_w, gu_s, mlp, g)   # gate|up projection with the SiLU * up epilogue
            else:
                _lib.silu_mul_f16(self._prefill_linear(h, gu_w, gu_s), mlp)
            nxt = self.layers[i + 1].input_norm if i + 1 < len(self.layers) else self.norm
            if t <= FUSED_PREFILL_NATIVE_MAX_ROWS:
                # down + residual add + the next norm (the op's K slices summed in the norm's launch)
                _lib.linear_add_rmsnorm_f16(mlp, b.down_proj.packed_weights, b.down_proj.scales, x, nxt.weight,
                                            nxt.eps, x, h, g)
            else:
                d = self._prefill_linear(mlp, b.down_proj.packed_weights, b.down_proj.scales)
                _lib.add_rmsnorm_f16(x, d, nxt.weight, nxt.eps, x, h)
        _lib.gemv_fused_f16(h[-1], self.lm_head.packed_weights, self.lm_head.scales, self.logits)
        _lib.argmax_embed_f16(self.logits, self.token, None, self.embed, self.x_buf)
        if not one_launch:
            self.position.fill_(t)

    def _prefill_linear(self, x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
        """A fused-prefill projection: the W4A16 op up to
        FUSED_PREFILL_NATIVE_MAX_ROWS rows, dequantize + hipBLASLt beyond."""
        if x.shape[0] <= FUSED_PREFILL_NATIVE_MAX_ROWS:
            return torch.ops.w4a16.linear(x, packed, scales, self.cfg.group_size)
        return F.linear(x, dequantize_cuda(packed, scales, self.cfg.group_size))

    @torch.inference_mode()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        """Run the prompt (int64 [T]); sets the next token and position; returns
        it. A prompt of the length captured by capture_prefill replays that graph."""
        if self.prefill_graph is not None and prompt.numel() == self.prefill_tokens.numel():
            self.prefill_tokens.copy_(prompt)
            self.prefill_graph.replay()
        else:
            self._prefill(prompt, torch.arange(prompt.numel(), device=prompt.device))
        self.host_position = prompt.numel()
        return self.token.clone()

    @torch.inference_mode()
    def capture_prefill(self, prompt_len: int) -> None:
        """Record prefill of a prompt_len-token prompt in a HIP graph (the
        prompt is copied into a static buffer before each replay). Sets the
        token and position like a prefill does; the torch-op prefill also
        resets the KV caches."""
        device = self.token.device
        # Every tensor the graph reads must outlive it: the token and position
        # buffers are attributes (a local allocated before the capture would be
        # freed on return and its memory reused under the recorded kernels).
        self.prefill_tokens = torch.zeros((prompt_len,), dtype=torch.int64, device=device)
        self.prefill_positions = torch.arange(prompt_len, device=device)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            self._prefill(self.prefill_tokens, self.prefill_positions)   # warm-up outside the capture
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._prefill(self.prefill_tokens, self.prefill_positions)
        torch.cuda.synchronize()
        self.prefill_graph = graph

    def short_step(self) -> bool:
        """Whether the next step (at host_position) takes the attention + o
        launch, which covers positions below 64."""
        return self.attn_o and self.host_position < min(64, self.cfg.max_seq_len)

    def _step(self, short: bool | None = None, token_copy: torch.Tensor | None = None) -> None:
        """One decode step; token_copy (an int64 element) also receives the
        new token."""
        if self.fused:
            self._step_fused(self.short_step() if short is None else short, token_copy)
            return
        logits = self._forward(self.token, self.position)
        self.logits.copy_(logits)
        self.token.copy_(torch.argmax(logits).view(1))
        self.position.add_(1)
        if token_copy is not None:
            token_copy.copy_(self.token[0])

    def _step_fused(self, short: bool = False, token_copy: torch.Tensor | None = None) -> None:
        """One decode step as 5 launches per layer plus 2 (include/w4a16_decode.h),
        4 per layer when `short` (attention + o projection in one launch; the
        position must then be below 64). x_buf holds the current token's
        embedding on entry (prefill gathers the first one); the final argmax
        gathers the next token's and writes the token to token_copy as well."""
        cfg = self.cfg
        x = self.x_buf
        for i, b in enumerate(self.layers):
            qkv_w, qkv_s = self.qkv[i]
            gu_w, gu_s = self.gate_up[i]
            if short and self.qkv_rope:
                _lib.gemv_qkv_rope_f16(x, qkv_w, qkv_s, self.qkv_buf, self.k_cache[i], self.v_cache[i],
                                       self.inv_freq, self.position, cfg.num_heads, cfg.num_kv_heads,
                                       norm_weight=b.input_norm.weight, eps=b.input_norm.eps)
                _lib.attention_o_cached_f16(self.qkv_buf, self.k_cache[i], self.v_cache[i], self.position,
                                            b.o_proj.packed_weights, b.o_proj.scales, x, cfg.num_heads,
                                            cfg.num_kv_heads, cfg.head_dim, cfg.group_size)
            elif short:
                _lib.gemv_fused_f16(x, qkv_w, qkv_s, self.qkv_buf, norm_weight=b.input_norm.weight,
                                    eps=b.input_norm.eps)
                _lib.attention_o_f16(self.qkv_buf, self.k_cache[i], self.v_cache[i], self.inv_freq, self.position,
                                     b.o_proj.packed_weights, b.o_proj.scales, x, cfg.num_heads, cfg.num_kv_heads,
                                     cfg.head_dim, cfg.group_size)
            else:
                _lib.gemv_fused_f16(x, qkv_w, qkv_s, self.qkv_buf, norm_weight=b.input_norm.weight,
                                    eps=b.input_norm.eps)
                if self.attn_splits:
                    _lib.decode_attention_split_f16(self.qkv_buf, self.k_cache[i], self.v_cache[i], self.cos,
                                                    self.sin, self.position, self.attn_buf, cfg.num_heads,
                                                    cfg.num_kv_heads, self.attn_splits, self.attn_ws, cfg.head_dim)
                else:
                    _lib.decode_attention_f16(self.qkv_buf, self.k_cache[i], self.v_cache[i], self.cos, self.sin,
                                              self.position, self.attn_buf, cfg.num_heads, cfg.num_kv_heads,
                                              cfg.head_dim)
                _lib.gemv_fused_f16(self.attn_buf, b.o_proj.packed_weights, b.o_proj.scales, x, residual=x)
            _lib.gemv_fused_f16(x, gu_w, gu_s, self.mlp_buf, norm_weight=b.post_norm.weight, eps=b.post_norm.eps,
                                paired=True)
            _lib.gemv_fused_f16(self.mlp_buf, b.down_proj.packed_weights, b.down_proj.scales, x, residual=x)
        # RMSNorm + lm_head GEMV, then greedy argmax + position += 1 + the next
        # token's embedding into x_buf. Two launches: the single-launch form
        # (w4a16_gemv_argmax_f16) pays one device-scope fence per workgroup.
        _lib.gemv_fused_f16(x, self.lm_head.packed_weights, self.lm_head.scales, self.logits,
                            norm_weight=self.norm.weight, eps=self.norm.eps)
        _lib.argmax_embed_f16(self.logits, self.token, self.position, self.embed, x, token_copy=token_copy)

    @torch.inference_mode()
    def step(self) -> torch.Tensor:
        """One eager decode step; returns the new token."""
        self._step()
        self.host_position += 1
        return self.token.clone()

    def _capture_step(self, short: bool) -> torch.cuda.CUDAGraph:
        """A decode step in a HIP graph, after a warm-up eager step on a side
        stream so lazy initialisation is not captured."""
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            self._step(short)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._step(short)
        torch.cuda.synchronize()
        return graph

    def _capture_steps(self, count: int) -> torch.cuda.CUDAGraph:
        """`count` short steps in one HIP graph, step j writing its token to
        multi_tokens[j] as well (a warm-up run on a side stream first)."""
        def steps():
            for j in range(count):
                self._step(True, self.multi_tokens[j:j + 1])

        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            steps()
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            steps()
        torch.cuda.synchronize()
        return graph

    @torch.inference_mode()
    def capture(self, tokens_per_replay: int = 1) -> None:
        """Record the decode step in HIP graphs: the general one and, when the
        attention + o launch applies, the step for positions below 64; with
        tokens_per_replay = T > 1 also graphs of T, T // 2, T // 4, .. (more
        than one) of those short steps, which `replay_tokens` uses while the
        position stays below 64, the largest that fits first (every graph
        replay costs a fixed 12-16 us of GPU time: 31 tokens at T = 16 take 5
        replays). The KV cache, position and the fused step's input row are
        restored afterwards (capturing runs steps)."""
        saved = (self.k_cache.clone(), self.v_cache.clone(), self.token.clone(), self.position.clone(),
                 self.x_buf.clone())

        def restore():
            self.k_cache.copy_(saved[0])
            self.v_cache.copy_(saved[1])
            self.token.copy_(saved[2])
            self.position.copy_(saved[3])
            self.x_buf.copy_(saved[4])

        self.graph = self._capture_step(False)
        restore()
        self.graph_multi = None
        self.graphs_multi = {}
        if self.attn_o:
            # the warm-up step must see a position the short step accepts
            short_end = min(64, self.cfg.max_seq_len)
            self.position.fill_(min(self.host_position, short_end - 1))
            self.graph_short = self._capture_step(True)
            restore()
            if tokens_per_replay > 1 and tokens_per_replay <= short_end:
                self.multi_tokens = torch.zeros((tokens_per_replay,), dtype=torch.int64, device=self.position.device)
                count = tokens_per_replay
                while count > 1:
                    # the capture runs 2 count steps (warm-up and recording) from a position they all accept
                    self.position.fill_(max(0, min(self.host_position, short_end - count)))
                    self.graphs_multi[count] = self._capture_steps(count)
                    restore()
                    count //= 2
                self.graph_multi = self.graphs_multi[tokens_per_replay]
        torch.cuda.synchronize()

    def replay(self) -> None:
        """One decode step: the captured graph for the current position."""
        assert self.graph is not None, "call capture() first"
        if self.graph_short is not None and self.short_step():
            self.graph_short.replay()
        else:
            self.graph.replay()
        self.host_position += 1

    def multi_steps(self, limit: int | None = None) -> int:
        """Steps of the largest multi-step graph that applies now: at most
        `limit` steps and none past position 63 (0 when none does)."""
        end = min(64, self.cfg.max_seq_len)
        fits = [c for c in self.graphs_multi if self.host_position + c <= end and (limit is None or c <= limit)]
        return max(fits, default=0)

    def replay_tokens(self, limit: int | None = None) -> torch.Tensor:
        """Replay decode graphs for the next tokens: the largest multi-step
        graph that applies with at most `limit` tokens, else one step. Returns
        the new tokens (int64 [n], on the device)."""
        t = self.multi_steps(limit)
        if t:
            self.graphs_multi[t].replay()
            self.host_position += t
            return self.multi_tokens[:t].clone()
        self.replay()
        return self.token.clone()

    @torch.inference_mode()
    def generate(self, prompt: torch.Tensor, new_tokens: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy decode: prefill, then new_tokens - 1 decode steps (several per
        graph replay when capture(tokens_per_replay > 1) recorded them)."""
        out = [self.prefill(prompt)]
        left = new_tokens - 1
        while left > 0:
            if use_graph:
                toks = self.replay_tokens(limit=left)
                out.append(toks)
                left -= toks.numel()
            else:
                out.append(self.step())
                left -= 1
        return torch.cat(out)
