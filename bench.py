"""Benchmark of the MI355X W4A16 linear layer (one GPU).

Metric: INT4 GEMV us & % of HBM peak per layer (M=1); decode
tok/s, 1.1B Llama.

Workload of the headline line (`value`, configs[1]): the two MLP layer shapes
at M = 1 -- up/gate K=2048 N=5632 and down K=5632 N=2048 -- group size 128,
fp16 activations ~N(0,1), weights ~N(0,0.02) fp32 quantized RTN absmax, each
shape with 64 rotated weight copies (762 MB together) so no layer runs from
the 256 MB Infinity Cache. One step = one call of each shape on its next
copy. 0.25 s of untimed graph replays of whole rotations bring the GPU out of
its idle clock; then untimed pre-roll replays (enough to keep the GPU busy
while the host enqueues the timed calls), the W warm-up steps (a graph) and
exactly K timed steps, enqueued as eager calls, go back to back, the K steps
bracketed by events on the stream (synchronised before and after). The GPU
must still be in the pre-roll when the last timed call is enqueued (checked:
the start event has not fired), so the events hold the 2K kernels and no host
launch gap; the same K steps replayed as one graph carry the graph launch's
own 9-10 us of GPU time and are reported beside it (`value_graph_replay`).
`value` = algorithmic bytes moved by the K steps / elapsed time (GB/s), with
algorithmic bytes per call N*K/2 + N*(K/128)*2 + M*K*2 + M*N*2 (reference
scripts/profile_kernel.py:310-323).

Rotation: step g reads copy g mod 64 of one continuous sequence -- an untimed
64-step pre-roll, the warm-up steps, the timed steps -- so every timed call
reads a copy last read 64 steps (762 MB of other weights) earlier.

Also reported: per-layer us / GB/s / % of the 8 TB/s HBM peak for each shape
(graph replay of whole rotations over the copies, at least 100 calls) with
the single-call eager latency (`eager_us`, launch included), GPU clocks and
power sampled under load, the configs[2] small-batch table (M = 1, 2, 4, 8
on 2048x2048, 2048x5632, 5632x2048, next to fp16 hipBLASLt on the dequantized
weights) and the configs[3] large-layer table (M = 1, 8), a measured device
copy bandwidth, end-to-end greedy decode tokens/s of the random-init 1.1B
Llama-architecture model (configs[4], decode step in a HIP graph), and the
CPU oracle's time for the same layers on the host cores (`cpu_baseline`; a
reported baseline, not a target), with configs[0] (M = 1, 2048 x 2048) timed
on the product's torch CPU path beside the oracle, and the CPU model.

Every leg runs inside a named roctx range (torch.cuda.nvtx on ROCm;
`rocprofv3 --marker-trace` records them), and `--profiler torch` writes a
Chrome trace of the configs[1] calls, as the reference's profiler script does.

usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-decode] [--no-cpu] [--no-tables] [--long]
                       [--profiler none|torch] [--trace-dir DIR]
       python bench.py --headline-pass | --layer-pass M K N COPIES CALLS | --prefill-pass TOKENS   (profiler passes)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
# Untimed back-to-back replays before the headline's timed steps: the GPU's
# clock rises from idle only under sustained load.
SETTLE_SECONDS = 0.25
# The same before each per-layer timing (whose weights the host has just
# built while the GPU idled).
LAYER_SETTLE_SECONDS = 0.15
# Most decode steps per graph replay in the decode measurement: the decoder
# captures graphs of 16, 8, 4 and 2 steps and the generation loop replays the
# largest that fits the tokens left while the position allows it, one step
# otherwise (31 tokens: 5 replays); the one-step-per-replay rate is reported
# beside it.
TOKENS_PER_REPLAY = 16
# HBM bytes per launch of the M=1 GEMV on the two configs[1] shapes (mean),
# from rocprofv3 FETCH_SIZE and WRITE_SIZE passes over `bench.py --counter-pass`,
# each scaled by the counter's reading on a kernel of known traffic (FETCH_SIZE
# reads half the bytes on this part, WRITE_SIZE is exact).
MEASURED_TRAFFIC_BYTES = 6141114
TRAFFIC_SOURCE = "profiles/gemv_pair_ring_m1_mlp_traffic.md"
# Mean kernel duration of the same two kernels in a rocprofv3 kernel trace of
# `bench.py --headline-pass` (the headline sequence alone, outside its timed
# steps), per launch; the line reports the trace's fraction beside the
# event-timed one.
TRACE_US_PER_LAUNCH = 3.064
TRACE_SOURCE = "profiles/gemv_pair_ring_m1_mlp_kernel_trace.md"


def _kernel_name(plan: dict, m: int = 1, k: int = 0) -> str:
    """Template instance the C ABI launches for a plan (w4a16_kernels.h,
    w4a16_pair_ring.h)."""
    if plan["kernel"] == "pair_ring":
        slots = 1 if m <= 1 else 4 if m <= 4 else 8
        pairs = -(-(k // 256) // max(1, plan["splits"]))
        return (f"w4a16::gemv_pair_ring<{slots},{plan['splits']},{plan['rows']},1,{pairs},"
                f"{plan['unroll']}>")
    if plan["kernel"] == "oneshot":
        return f"w4a16::gemv_oneshot<1,{plan['rows']},{plan['unroll']},{plan['splits']}>"
    if plan["kernel"] == "valu":
        return f"w4a16::gemv_valu<1,{plan['rows']},{plan['unroll']},false>"
    return f"w4a16 {plan['kernel']} kernel"


def torch_inference(fn):
    """fn under torch.inference_mode (the decoder's buffers are inference
    tensors; graph captures of launches on them must run in that mode)."""
    def wrapped(*args, **kwargs):
        import torch

        with torch.inference_mode():
            return fn(*args, **kwargs)

    return wrapped


class trace_range:
    """A named range around one leg of the bench (reference
    scripts/profile_kernel.py:346-352 wraps each baseline in an NVTX range):
    torch.cuda.nvtx is roctx on ROCm, so `rocprofv3 --marker-trace` records
    it and the kernels inside the range's span belong to that leg."""

    def __init__(self, name: str):
        self.name = name

    def __enter__(self):
        import torch

        torch.cuda.nvtx.range_push(self.name)
        return self

    def __exit__(self, *exc):
        import torch

        torch.cuda.nvtx.range_pop()
        return False


def torch_trace(op, iters: int, path: str) -> None:
    """Chrome trace of `iters` eager calls of `op` (reference
    scripts/profile_kernel.py:576-591, its --profiler torch)."""
    import torch

    os.makedirs(os.path.dirname(path) or ".", exist_ok=True)
    activities = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    with torch.profiler.profile(activities=activities, record_shapes=True) as prof:
        for i in range(iters):
            op(i)
        torch.cuda.synchronize()
    prof.export_chrome_trace(path)


def payload_bytes(m: int, n: int, k: int, group: int = 128) -> int:
    return n * k // 2 + n * (k // group) * 2 + m * k * 2 + m * n * 2


def make_layer(k: int, n: int, copies: int, device, seed: int = 0):
    import torch

    from nibble_amd.quantization import quantize_and_pack_weights

    gen = torch.Generator(device=device).manual_seed(seed)
    w = torch.randn((n, k), device=device, generator=gen) * 0.02
    packed, scales = quantize_and_pack_weights(w, 128)
    del w
    return [packed.clone() for _ in range(copies)], [scales.clone() for _ in range(copies)]


def capture(fn, count: int):
    import torch

    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn(0)  # warm any lazy state outside the capture
        with torch.cuda.graph(graph, stream=stream):
            for i in range(count):
                fn(i)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    return graph


def time_graph(graph, reps: int = 1) -> float:
    """Seconds for `reps` replays, events on the replay (current) stream."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def per_layer(op, copies: int, calls: int = 100, samples: int = 20) -> float:
    """Median microseconds per call over `samples` replays of a graph of at
    least `calls` calls over the rotated copies, after LAYER_SETTLE_SECONDS of
    untimed replays. The graph holds whole rotations (a multiple of `copies`
    calls), so across replays as within one every copy is read again only
    after all the other copies were."""
    import torch

    calls = copies * -(-calls // copies)
    graph = capture(lambda i: op(i % copies), calls)
    # untimed replays until the GPU has left the clock it idled at while the
    # host built the weights (as the headline's settle does)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < LAYER_SETTLE_SECONDS:
        for _ in range(5):
            graph.replay()
        torch.cuda.synchronize()
    times = sorted(time_graph(graph) / calls * 1e6 for _ in range(samples))
    return times[len(times) // 2]


def eager_us(op, copies: int, samples: int = 20) -> float:
    """Single-call latency with launch overhead (reference
    scripts/profile_kernel.py:531-534): events around one eager call, median
    over `samples` calls on successive rotated copies."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    times = []
    for i in range(samples):
        torch.cuda.synchronize()
        start.record()
        op(i % copies)
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3)
    times.sort()
    return times[len(times) // 2]


def gpu_state_under_load(graph, seconds: float = 1.0) -> dict | None:
    """GFX / memory clocks and socket power sampled with amdsmi while `graph`
    replays back to back, 20 replays per host wait (the counterpart of reference
    scripts/profile_kernel.py:256-307); None when amdsmi is unavailable."""
    import threading

    import torch

    try:
        import amdsmi

        amdsmi.amdsmi_init()
    except Exception:
        return None
    samples, stop = [], threading.Event()

    def sampler(handle):
        while not stop.is_set():
            try:
                gfx = amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.GFX)
                mem = amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.MEM)
                power = amdsmi.amdsmi_get_power_info(handle)
                watts = power.get("socket_power")
                if not isinstance(watts, (int, float)):
                    watts = power.get("current_socket_power")
                samples.append((gfx.get("clk"), mem.get("clk"), watts))
            except Exception:
                pass
            stop.wait(0.05)

    firmware = {}
    try:
        handles = amdsmi.amdsmi_get_processor_handles()
        if not handles:
            return None
        try:
            # The compute microcode (MEC) decides whether kernel arguments are
            # preloaded into SGPRs or loaded by the code object's prologue.
            for entry in amdsmi.amdsmi_get_fw_info(handles[0]).get("fw_list", []):
                name = str(entry.get("fw_name", entry.get("fw_id", "")))
                if "MEC" in name or "RLC" in name:
                    firmware[name.split(".")[-1]] = str(entry.get("fw_version"))
        except Exception:
            pass
        thread = threading.Thread(target=sampler, args=(handles[0],), daemon=True)
        thread.start()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            for _ in range(20):
                graph.replay()
            torch.cuda.synchronize()
        stop.set()
        thread.join()
    finally:
        stop.set()
        try:
            amdsmi.amdsmi_shut_down()
        except Exception:
            pass

    def stats(values):
        vals = [v for v in values if isinstance(v, (int, float)) and v not in (0xFFFF, 0xFFFFFFFF)]
        if not vals:
            return None
        vals.sort()
        return {"min": vals[0], "median": vals[len(vals) // 2], "max": vals[-1]}

    return {"samples": len(samples), "gfx_clock_mhz": stats([s[0] for s in samples]),
            "mem_clock_mhz": stats([s[1] for s in samples]), "socket_power_w": stats([s[2] for s in samples]),
            "firmware": firmware or None}


def copy_bandwidth(device) -> float:
    """Device-to-device copy of 1 GiB (read + write bytes / time), GB/s."""
    import torch

    a = torch.empty(1 << 28, dtype=torch.float32, device=device)
    b = torch.empty_like(a)
    graph = capture(lambda i: b.copy_(a), 5)
    graph.replay()
    t = min(time_graph(graph) for _ in range(3))
    del a, b
    return 2 * (1 << 30) * 5 / t / 1e9


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_call_us(fn, budget_s: float) -> tuple[float, int]:
    """Median wall time of fn() in microseconds over calls filling budget_s
    (after one warm-up call), and the number of timed calls."""
    fn()
    times = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or len(times) < 5:
        t1 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t1)
    times.sort()
    return times[len(times) // 2] * 1e6, len(times)


def cpu_baseline(shapes, budget_s: float = 12.0, port_budget_s: float = 6.0, configs0_budget_s: float = 3.0) -> dict:
    """The reference's CPU path (w4a16/reference.py:49-80: fp32 dequantize of
    the whole matrix, fp32 matmul, fp16 cast), as the product's torch
    restatement nibble_amd.reference.linear_reference (which QuantizedLinear
    runs for CPU tensors), timed on the host cores on a bounded sample of the
    same layers (M = 1, one weight copy per shape): `value`. Beside it the C
    oracle (the same arithmetic with float64 sums, OpenMP) on the same layers,
    and configs[0] (M = 1, 2048 x 2048) on both."""
    import numpy as np
    import torch

    import oracle
    from nibble_amd.reference import linear_reference

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    rng = np.random.default_rng(0)
    layers = []
    for k, n in shapes:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        packed, scales = oracle.quantize_and_pack(w, 128)
        x = rng.standard_normal((1, k)).astype(np.float16)
        layers.append((x, packed, scales, payload_bytes(1, n, k)))
    for x, p, s, _ in layers:  # warm-up
        oracle.linear(x, p, s, 128, threads=threads)
    calls, total_bytes = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < port_budget_s:
        for x, p, s, nbytes in layers:
            oracle.linear(x, p, s, 128, threads=threads)
            calls += 1
            total_bytes += nbytes
    port_elapsed = time.perf_counter() - t0

    # the reference's path in torch on the same layers and threads
    tlayers = [(torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(s), nbytes) for x, p, s, nbytes in layers]
    torch_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        for x, p, s, _ in tlayers:  # warm-up
            linear_reference(x, p, s, 128)
        ref_calls, ref_bytes = 0, 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            for x, p, s, nbytes in tlayers:
                linear_reference(x, p, s, 128)
                ref_calls += 1
                ref_bytes += nbytes
        ref_elapsed = time.perf_counter() - t0
    finally:
        torch.set_num_threads(torch_threads)

    # seed 0, weights randn(N, K) * 0.02 fp32 -> RTN group 128,
    # activations randn(1, K) -> fp16, as BASELINE.json states it
    k0 = n0 = 2048
    gen = torch.Generator().manual_seed(0)
    w0 = torch.randn((n0, k0), generator=gen) * 0.02
    from nibble_amd.quantization import quantize_and_pack_weights

    p0, s0 = quantize_and_pack_weights(w0, 128)
    x0 = torch.randn((1, k0), generator=gen).to(torch.float16)
    torch.set_num_threads(threads)
    try:
        torch_us, torch_calls = _median_call_us(lambda: linear_reference(x0, p0, s0, 128), configs0_budget_s)
    finally:
        torch.set_num_threads(torch_threads)
    xn, pn, sn = x0.numpy(), p0.numpy(), s0.numpy()
    port_us, port_calls = _median_call_us(lambda: oracle.linear(xn, pn, sn, 128, threads=threads),
                                          configs0_budget_s)
    b0 = payload_bytes(1, n0, k0)
    return {
        "value": round(ref_bytes / ref_elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference",
        "sample": f"{ref_calls} single-token calls alternating up (2048x5632) and down (5632x2048) "
                  f"in {ref_elapsed:.1f} s, 1 weight copy per shape, through the reference's CPU path "
                  f"(reference w4a16/reference.py:49-80 as nibble_amd.reference.linear_reference, torch CPU, "
                  f"{threads} threads)",
        "us_per_call": round(ref_elapsed / ref_calls * 1e6, 1),
        "port_value": round(total_bytes / port_elapsed / 1e9, 3),
        "port_us_per_call": round(port_elapsed / calls * 1e6, 1),
        "port": f"oracle.linear (C restatement, OpenMP, {threads} threads) on the same layers: {calls} calls in "
                f"{port_elapsed:.1f} s",
        "cpu_model": _cpu_model(),
        "logical_cpus": os.cpu_count(),
        "configs0": {
            "workload": "configs[0]: M=1 K=2048 N=2048 group 128, the reference's CPU path",
            "torch_reference_us": round(torch_us, 1),
            "torch_reference_GBps": round(b0 / torch_us / 1e3, 3),
            "torch_reference": f"nibble_amd.reference.linear_reference (torch CPU, {threads} threads), "
                               f"median of {torch_calls} calls",
            "port_us": round(port_us, 1),
            "port_GBps": round(b0 / port_us / 1e3, 3),
            "port": f"oracle.linear (C, OpenMP, {threads} threads), median of {port_calls} calls",
        },
    }


def decode_tok_s(device, runs: int = 5, new_tokens: int = 32, prompt_len: int = 16) -> dict:
    """greedy decode on the random-init 1.1B Llama, decode step in a
    HIP graph: the fused step (5 launches per layer) and, on the same weights,
    the step as separate torch ops around QuantizedLinear."""
    import torch

    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(max_seq_len=prompt_len + new_tokens)
    model = LlamaDecoder(cfg, device=device, seed=0)
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,), generator=gen).to(device)

    def timed(fused: bool, per_replay: int = 1):
        # as the reference's benchmark_prompt (scripts/generate.py:331-352):
        # the prefill timed on its own runs back to back (its
        # generate(max_new_tokens=1) samples), then the decode of the
        # new_tokens - 1 further tokens after an untimed prefill
        model.fused = fused
        model.prefill(prompt)
        model.capture(tokens_per_replay=per_replay)
        decode_s, prefill_s = [], []
        for _ in range(runs + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            model.prefill(prompt)
            torch.cuda.synchronize()
            prefill_s.append(time.perf_counter() - t0)
        for _ in range(runs + 1):
            model.prefill(prompt)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            left = new_tokens - 1
            while left > 0:
                left -= model.replay_tokens(limit=left).numel()
            torch.cuda.synchronize()
            decode_s.append(time.perf_counter() - t1)
        decode_s, prefill_s = sorted(decode_s[1:]), sorted(prefill_s[1:])
        return decode_s[len(decode_s) // 2], prefill_s[len(prefill_s) // 2]

    unfused_s, prefill_eager = timed(False)
    model.fused = True   # the prefill graph records the fused prefill
    model.capture_prefill(prompt_len)
    single, _ = timed(True)
    med, prefill = timed(True, TOKENS_PER_REPLAY)
    return {
        "decode_tok_s": round((new_tokens - 1) / med, 1),
        "ms_per_token": round(med / (new_tokens - 1) * 1e3, 3),
        "tokens_per_replay": TOKENS_PER_REPLAY,
        "decode_tok_s_one_step_per_replay": round((new_tokens - 1) / single, 1),
        "weight_GBps": round(model.packed_bytes() * (new_tokens - 1) / med / 1e9, 1),
        "step": "fused, positions < 64: RMSNorm+qkv GEMV+rotary+KV append, attention+o GEMV+residual, "
                "RMSNorm+gate|up GEMV+SiLU*up, down GEMV+residual per layer; RMSNorm+lm_head GEMV, argmax; "
                f"graphs of {TOKENS_PER_REPLAY}, {TOKENS_PER_REPLAY // 2}, .. 2 steps (the largest that fits the "
                "tokens left) while the position allows, else one step per replay",
        "unfused_decode_tok_s": round((new_tokens - 1) / unfused_s, 1),
        "prefill_ms": round(prefill * 1e3, 3),
        "prefill_timing": "host wall time of prefill() (the prompt copy, the graph replay, the token read-back) "
                          "and a synchronize, median of back-to-back runs, as the reference times its "
                          "generate(max_new_tokens=1) samples",
        "prefill_eager_ms": round(prefill_eager * 1e3, 3),
        "prefill": "16-token prompt, one HIP graph: the embeddings and their RMSNorm, then per layer the W4A16 op "
                   "for q|k|v (the ring kernel's 16-row-slot form), rotary + KV append + causal attention inside "
                   "the o projection's launch (8 K slices of 4 heads), the slices' sum + residual add + RMSNorm, "
                   "gate|up with the SiLU*up epilogue, down (8 K slices), the slices' sum + residual add + next "
                   "RMSNorm; then the lm_head GEMV on the last row and the argmax + next embedding; "
                   "prefill_eager_ms: the same prompt as eager torch ops around QuantizedLinear",
        "linear_layers": len(model.linear_layers()),
        "packed_weight_bytes_per_token": model.packed_bytes(),
        "model": "random-init Llama 22L h2048 i5632 32q/4kv hd64 vocab32000, INT4 g128 on all 155 linears",
        "prompt_tokens": prompt_len,
        "new_tokens": new_tokens,
    }


@torch_inference
def launch_times(device, prompt_len: int = 16) -> dict:
    """Per-launch GPU time of the configs[4] decoder's fused prefill (16
    tokens) and fused decode step: each launch kind captured 22 times (layer
    i's weights and caches in call i) in one graph, median replay time / 22,
    after untimed replays; the whole prefill graph timed with events around
    its replay. Inputs are the decoder's own buffers after a prefill (the
    values only set the data the launches read)."""
    import torch

    from nibble_amd import _lib
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    model = LlamaDecoder(LlamaConfig(max_seq_len=48), device=device, seed=0)
    cfg, g = model.cfg, model.cfg.group_size
    prompt = torch.randint(0, cfg.vocab_size, (prompt_len,), generator=torch.Generator().manual_seed(0)).to(device)
    model.capture_prefill(prompt_len)
    model.prefill(prompt)
    torch.cuda.synchronize()

    def graph_us(fn, count: int) -> float:
        graph = capture(lambda i: fn(i), count)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < LAYER_SETTLE_SECONDS:
            graph.replay()
            torch.cuda.synchronize()
        times = sorted(time_graph(graph) for _ in range(15))
        return times[len(times) // 2] / count * 1e6

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    whole = []
    for _ in range(15):
        torch.cuda.synchronize()
        start.record()
        model.prefill_graph.replay()
        end.record()
        end.synchronize()
        whole.append(start.elapsed_time(end) * 1e3)
    whole.sort()
    layers = len(model.layers)
    x = model.embed[prompt].contiguous()
    h = torch.empty_like(x)
    qkv = torch.empty((prompt_len, model.qkv[0][0].shape[0]), dtype=torch.float16, device=device)
    mlp = torch.empty((prompt_len, cfg.intermediate_size), dtype=torch.float16, device=device)
    blk = model.layers
    prefill = {
        "embedding rows + RMSNorm + position (once)": lambda i: _lib.embed_rmsnorm_f16(
            model.embed, model.prefill_tokens, blk[0].input_norm.weight, 1e-5, x, h),
        "q|k|v op": lambda i: _lib.linear_f16(h, model.qkv[i][0], model.qkv[i][1], qkv),
        "attention + o op, then slice sum + residual + RMSNorm (2 launches)":
            lambda i: _lib.prefill_attention_o_add_rmsnorm_f16(
                qkv, model.k_cache[i], model.v_cache[i], model.cos, model.sin, 0, blk[i].o_proj.packed_weights,
                blk[i].o_proj.scales, x, blk[i].post_norm.weight, 1e-5, x, h, cfg.num_heads, cfg.num_kv_heads,
                cfg.head_dim, g),
        "gate|up op + SiLU * up": lambda i: _lib.linear_silu_f16(h, model.gate_up[i][0], model.gate_up[i][1], mlp, g),
        "down op, then slice sum + residual + RMSNorm (2 launches)":
            lambda i: _lib.linear_add_rmsnorm_f16(mlp, blk[i].down_proj.packed_weights, blk[i].down_proj.scales, x,
                                                  blk[i].post_norm.weight, 1e-5, x, h, g),
        "lm_head GEMV (once)": lambda i: _lib.gemv_fused_f16(h[-1], model.lm_head.packed_weights,
                                                             model.lm_head.scales, model.logits),
        "argmax + next embedding (once)": lambda i: _lib.argmax_embed_f16(model.logits, model.token, None,
                                                                          model.embed, model.x_buf),
    }
    out = {"prefill_tokens": prompt_len,
           "prefill_graph_us": round(whole[len(whole) // 2], 2),
           "prefill_us_per_launch": {k: round(graph_us(f, layers), 2) for k, f in prefill.items()}}
    # the decode step's launches at position 16 (below 64: the short step)
    model.position.fill_(prompt_len)
    xb = model.x_buf
    step = {
        "RMSNorm + q|k|v GEMV + rotary + KV append": lambda i: _lib.gemv_qkv_rope_f16(
            xb, model.qkv[i][0], model.qkv[i][1], model.qkv_buf, model.k_cache[i], model.v_cache[i], model.inv_freq,
            model.position, cfg.num_heads, cfg.num_kv_heads, norm_weight=blk[i].input_norm.weight, eps=1e-5),
        "attention + o GEMV + residual": lambda i: _lib.attention_o_cached_f16(
            model.qkv_buf, model.k_cache[i], model.v_cache[i], model.position, blk[i].o_proj.packed_weights,
            blk[i].o_proj.scales, xb, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, g),
        "RMSNorm + gate|up GEMV + SiLU * up": lambda i: _lib.gemv_fused_f16(
            xb, model.gate_up[i][0], model.gate_up[i][1], model.mlp_buf, norm_weight=blk[i].post_norm.weight,
            eps=1e-5, paired=True),
        "down GEMV + residual": lambda i: _lib.gemv_fused_f16(model.mlp_buf, blk[i].down_proj.packed_weights,
                                                              blk[i].down_proj.scales, xb, residual=xb),
        "RMSNorm + lm_head GEMV (once)": lambda i: _lib.gemv_fused_f16(
            xb, model.lm_head.packed_weights, model.lm_head.scales, model.logits, norm_weight=model.norm.weight,
            eps=1e-5),
        "argmax + next embedding (once)": lambda i: _lib.argmax_embed_f16(model.logits, model.token, None,
                                                                          model.embed, xb),
    }
    out["decode_us_per_launch"] = {k: round(graph_us(f, layers), 2) for k, f in step.items()}
    return out


def decode_long_context(device, prompt_len: int = 1500, max_seq_len: int = 2048, new_tokens: int = 64,
                        runs: int = 3) -> dict:
    """Graph-replayed decode (one step per replay: positions past 63) after a 1500-token prompt
    in a 2048-slot cache on the random-init 1.1B Llama: the decode attention
    split over the slots (the decoder's default past 512 slots) against one
    workgroup per head."""
    import torch

    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    model = LlamaDecoder(LlamaConfig(max_seq_len=max_seq_len), device=device, seed=0)
    prompt = torch.randint(0, model.cfg.vocab_size, (prompt_len,), generator=torch.Generator().manual_seed(2))
    prompt = prompt.to(device)
    splits = model.attn_splits

    def timed() -> float:
        model.prefill(prompt)
        model.capture(tokens_per_replay=TOKENS_PER_REPLAY)
        ts = []
        for _ in range(runs + 1):
            model.prefill(prompt)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            left = new_tokens
            while left > 0:
                left -= model.replay_tokens(limit=left).numel()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        ts = sorted(ts[1:])
        return new_tokens / ts[len(ts) // 2]

    split_rate = timed()
    model.attn_splits = 0
    single_rate = timed()
    del model
    torch.cuda.empty_cache()
    return {f"decode_ctx{prompt_len}_tok_s": round(split_rate, 1),
            f"decode_ctx{prompt_len}_one_wg_per_head_tok_s": round(single_rate, 1),
            "decode_long_context": f"{new_tokens} tokens after a {prompt_len}-token prompt, {max_seq_len}-slot "
                                   f"cache, one step per graph replay: decode attention split "
                                   f"into {splits} shares per head, against one workgroup per head"}


def prefill_long(device, lengths=(64, 256, 1024), runs: int = 5) -> dict:
    """Prompts of 64, 256 and 1024 tokens on the random-init 1.1B Llama, each
    path recorded in a HIP graph: the fused prefill (every projection on the
    W4A16 op: its GEMM at M = 64, the LDS-staged and 32x32 GEMMs above; the
    1024-token attention streams the caches through LDS in 256-slot blocks)
    against the reference's prefill path (every projection as dequantize +
    hipBLASLt inside QuantizedLinear, torch ops around them)."""
    import torch

    from nibble_amd.linear import FUSED_MAX_ROWS, NATIVE_GEMM_MAX_ROWS
    from nibble_amd.llama import LlamaConfig, LlamaDecoder

    model = LlamaDecoder(LlamaConfig(max_seq_len=max(lengths)), device=device, seed=0)
    gen = torch.Generator().manual_seed(1)
    result = {}
    for prompt_len in lengths:
        prompt = torch.randint(0, model.cfg.vocab_size, (prompt_len,), generator=gen).to(device)

        def timed() -> float:
            model.capture_prefill(prompt_len)
            ts = []
            for _ in range(runs + 1):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                model.prefill(prompt)
                torch.cuda.synchronize()
                ts.append(time.perf_counter() - t0)
            ts = sorted(ts[1:])
            return ts[len(ts) // 2]

        model.fused = True
        for b in model.layers:
            b.native_prefill = True
        fused = timed()
        model.fused = False
        for b in model.layers:
            b.native_prefill = False
        for mod in model.linear_layers():   # the reference's routing: dequantize + GEMM for every M > 8
            mod.native_max_rows = FUSED_MAX_ROWS
        dequant = timed()
        for mod in model.linear_layers():
            mod.native_max_rows = NATIVE_GEMM_MAX_ROWS
        result[f"prefill{prompt_len}_ms"] = round(fused * 1e3, 3)
        result[f"prefill{prompt_len}_dequant_ms"] = round(dequant * 1e3, 3)
    model.prefill_graph = None
    del model
    torch.cuda.empty_cache()
    result["prefill_long"] = ("prompts of " + " and ".join(str(n) for n in lengths) + " tokens, one HIP graph "
                              "each: the fused prefill (W4A16 GEMM for q|k|v, o, gate|up, down) against dequantize "
                              "+ hipBLASLt for every projection with torch ops around them (the reference's "
                              "prefill path)")
    return result


def _copies(nbytes: int, floor_bytes: int = 512 << 20) -> int:
    """Rotated copies so the working set is >= 2x the 256 MiB Infinity Cache."""
    return max(2, -(-floor_bytes // nbytes))


def row_metrics(m: int, n: int, k: int, us: float, copy_gbps: float | None) -> dict:
    """us, GB/s, % of the 8 TB/s peak, % of the measured copy bandwidth and
    arithmetic intensity (FLOP per algorithmic byte) of one layer call, as the
    reference reports them per row (scripts/profile_kernel.py:622-628)."""
    gbs = payload_bytes(m, n, k) / us / 1e3
    row = {"us": round(us, 3), "GBps": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBPS, 2)}
    if copy_gbps:
        row["pct_copy"] = round(100 * gbs / copy_gbps, 2)
    row["flop_per_byte"] = round(2 * m * n * k / payload_bytes(m, n, k), 2)
    return row


def layer_tables(device, copy_gbps: float | None = None) -> dict:
    """M in {1, 2, 4, 8} on the three small-batch shapes, each next
    to an fp16 hipBLASLt GEMM (F.linear) on the dequantized weights; configs[3]:
    the 8B- and 70B-class shapes at M in {1, 8}. Per-layer time = median of
    graph replays of 100 calls over rotated weight copies."""
    import torch
    import torch.nn.functional as F

    from nibble_amd import _lib

    def rows_for(shapes, ms, with_fp16: bool, samples: int):
        rows = []
        for k, n in shapes:
            copies = _copies(n * k // 2)
            packed, scales = make_layer(k, n, copies, device, seed=k + n)
            w16 = []
            if with_fp16:
                c16 = _copies(2 * n * k)
                w16 = [torch.ops.w4a16.dequantize(packed[i % copies], scales[i % copies], 128) for i in range(c16)]
            base_us = None
            for m in ms:
                x = torch.randn((m, k), device=device).to(torch.float16)
                out = torch.empty((m, n), device=device, dtype=torch.float16)
                with trace_range(f"w4a16_fused M={m} K{k}xN{n}"):
                    us = per_layer(lambda i: _lib.linear_f16(x, packed[i], scales[i], out), copies, samples=samples)
                # the calls take a workspace from the caching allocator where the
                # plan uses one (the split-K routes), as the torch op does
                plan = _lib.plan_linear(x.data_ptr(), packed[0].data_ptr(), m, n, k, workspace=True)
                kernel = plan["kernel"] + (f" x{plan['max_blocks']} K slices"
                                           if plan["kernel"] == "pair_ring" and plan["max_blocks"] > 1 else "")
                row = {"K": k, "N": n, "M": m, **row_metrics(m, n, k, us, copy_gbps), "kernel": kernel,
                       "eager_us": round(eager_us(lambda i: torch.ops.w4a16.linear(x, packed[i], scales[i], 128),
                                                  copies), 3)}
                if m == 1:
                    base_us = us
                else:
                    row["vs_M1"] = round(us / base_us, 3)
                if w16:
                    with trace_range(f"w4a16_fp16 M={m} K{k}xN{n}"):
                        row["fp16_hipblaslt_us"] = round(
                            per_layer(lambda i: F.linear(x, w16[i]), len(w16), samples=samples), 3)
                    # the reference's dequant_every_call baseline: the weights
                    # dequantized on every call (here by the dequantize op),
                    # then the fp16 GEMM
                    with trace_range(f"w4a16_dequant M={m} K{k}xN{n}"):
                        row["dequant_every_call_us"] = round(per_layer(
                            lambda i: F.linear(x, torch.ops.w4a16.dequantize(packed[i], scales[i], 128)), copies,
                            samples=samples), 3)
                rows.append(row)
            del packed, scales, w16
            torch.cuda.empty_cache()
        return rows

    small = rows_for([(2048, 2048), (2048, 5632), (5632, 2048)], (1, 2, 4, 8), True, 10)
    large = rows_for([(4096, 4096), (4096, 14336), (14336, 4096), (8192, 8192), (8192, 28672), (28672, 8192)],
                     (1, 8), False, 5)
    return {"configs2_small_batch": small, "configs3_large": large}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-tables", action="store_true", help="skip the configs[2] / configs[3] per-layer tables")
    ap.add_argument("--long", action="store_true",
                    help="also time prompts of 64 / 256 / 1024 tokens and decode after a 1500-token prompt (no "
                         "BASELINE config covers them)")
    ap.add_argument("--profiler", choices=("none", "torch"), default="none",
                    help="torch: also write a Chrome trace of 20 torch-op calls of each configs[1] shape to "
                         "--trace-dir (reference scripts/profile_kernel.py --profiler torch)")
    ap.add_argument("--trace-dir", default="profile_results", help="directory of the --profiler torch traces")
    ap.add_argument("--headline-pass", action="store_true",
                    help="for rocprofv3 --kernel-trace: the headline sequence alone (clock settle, pre-roll, "
                         "warm-up, the K timed eager steps); prints the event-timed ms per step; no JSON")
    ap.add_argument("--counter-pass", action="store_true",
                    help="eager launches only, for rocprofv3 --pmc: 50 calls of each MLP shape on rotated "
                         "copies, then 5 elementwise negations of a 256 MiB fp32 buffer into another "
                         "(256 MiB read + 256 MiB written each: the byte-count calibration); no JSON")
    ap.add_argument("--layer-pass", type=int, nargs=5, metavar=("M", "K", "N", "COPIES", "CALLS"),
                    help="eager launches only, for rocprofv3 --pmc: CALLS default-dispatch calls of one "
                         "[M, K] x [N, K] layer on COPIES rotated weight copies; no JSON")
    ap.add_argument("--prefill-pass", type=int, metavar="TOKENS",
                    help="for rocprofv3 --kernel-trace: capture the fused prefill of a TOKENS-token prompt on the "
                         "random-init 1.1B Llama and replay it 10 times; no JSON")
    ap.add_argument("--launch-pass", action="store_true",
                    help="graph timing of each launch of the configs[4] decoder alone (the 16-token prefill's "
                         "and the decode step's), 22 launches per graph over the layers' weights, the "
                         "whole prefill graph beside them (rocprofv3 durations of graph-replayed kernels run "
                         "above these); prints one JSON line")
    ap.add_argument("--decode-pass", type=int, nargs=2, metavar=("CONTEXT", "SPLITS"),
                    help="for rocprofv3 --kernel-trace: on the random-init 1.1B Llama with a 2048-slot cache, "
                         "prefill a CONTEXT-token prompt, then decode 64 tokens by graph replay (one step per "
                         "replay) with the decode attention split into SPLITS shares per head (0: one workgroup "
                         "per head, -1: the decoder's default); no JSON")
    ap.add_argument("--decode-step-pass", action="store_true",
                    help="for rocprofv3 --kernel-trace: the decode leg's fused measurement alone (configs[4]: "
                         "random-init 1.1B Llama, 48-slot cache, 16-token prompt, 31 tokens by replays of the "
                         f"{TOKENS_PER_REPLAY}, 8, 4, 2 and 1-step graphs, 6 times); no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import torch

    import nibble_amd
    from nibble_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if not nibble_amd.cuda_extension_available():
        raise RuntimeError(f"W4A16 HIP extension not loaded: {nibble_amd.cuda.extension_load_error()}")
    device = torch.device("cuda:0")
    torch.manual_seed(0)

    if args.prefill_pass:
        from nibble_amd.llama import LlamaConfig, LlamaDecoder

        t = args.prefill_pass
        model = LlamaDecoder(LlamaConfig(max_seq_len=max(48, t)), device=device, seed=0)
        prompt = torch.randint(0, model.cfg.vocab_size, (t,), generator=torch.Generator().manual_seed(0)).to(device)
        model.capture_prefill(t)
        torch.cuda.synchronize()
        for _ in range(10):
            model.prefill(prompt)
        torch.cuda.synchronize()
        print("prefill pass done", flush=True)
        return 0

    if args.launch_pass:
        print(json.dumps(launch_times(device)), flush=True)
        return 0

    if args.decode_step_pass:
        from nibble_amd.llama import LlamaConfig, LlamaDecoder

        prompt_len, new_tokens = 16, 32
        model = LlamaDecoder(LlamaConfig(max_seq_len=prompt_len + new_tokens), device=device, seed=0)
        prompt = torch.randint(0, model.cfg.vocab_size, (prompt_len,), generator=torch.Generator().manual_seed(0))
        prompt = prompt.to(device)
        model.prefill(prompt)
        model.capture(tokens_per_replay=TOKENS_PER_REPLAY)
        for _ in range(6):
            model.prefill(prompt)
            left = new_tokens - 1
            while left > 0:
                left -= model.replay_tokens(limit=left).numel()
        torch.cuda.synchronize()
        print("decode step pass done", flush=True)
        return 0

    if args.decode_pass:
        from nibble_amd.llama import LlamaConfig, LlamaDecoder

        ctx, splits = args.decode_pass
        model = LlamaDecoder(LlamaConfig(max_seq_len=2048), device=device, seed=0)
        if splits >= 0:
            model.attn_splits = splits
            model.attn_ws = torch.empty((max(1, model.cfg.num_heads * splits * 66),), dtype=torch.float32,
                                        device=device)
        prompt = torch.randint(0, model.cfg.vocab_size, (ctx,), generator=torch.Generator().manual_seed(0))
        model.prefill(prompt.to(device))
        model.capture(tokens_per_replay=TOKENS_PER_REPLAY)
        left = 64
        while left > 0:
            left -= model.replay_tokens(limit=left).numel()
        torch.cuda.synchronize()
        print("decode pass done", flush=True)
        return 0

    if args.layer_pass:
        m, k, n, lcopies, calls = args.layer_pass
        packed, scales = make_layer(k, n, lcopies, device, seed=0)
        x = torch.randn((m, k), device=device).to(torch.float16)
        out = torch.empty((m, n), device=device, dtype=torch.float16)
        torch.cuda.synchronize()
        for i in range(calls):
            _lib.linear_f16(x, packed[i % lcopies], scales[i % lcopies], out)
        torch.cuda.synchronize()
        print("layer pass done", flush=True)
        return 0

    copies = 64
    shapes = [(2048, 5632), (5632, 2048)]  # (K, N): up/gate and down
    layers = [make_layer(k, n, copies, device, seed=i) for i, (k, n) in enumerate(shapes)]
    xs = [torch.randn((1, k), device=device).to(torch.float16) for k, _ in shapes]
    outs = [torch.empty((1, n), device=device, dtype=torch.float16) for _, n in shapes]

    def call(j: int, i: int) -> None:
        packed, scales = layers[j]
        torch.ops.w4a16.linear(xs[j], packed[i % copies], scales[i % copies], 128)

    def call_raw(j: int, i: int) -> None:
        packed, scales = layers[j]
        _lib.linear_f16(xs[j], packed[i % copies], scales[i % copies], outs[j])

    if args.counter_pass:
        for i in range(50):
            call_raw(0, i)
            call_raw(1, i)
        a = torch.ones(1 << 26, dtype=torch.float32, device=device)
        b = torch.empty_like(a)
        for _ in range(5):
            torch.neg(a, out=b)
        torch.cuda.synchronize()
        print("counter pass done", flush=True)
        return 0

    # ---- headline: K timed steps (one call of each MLP shape per step) ----
    # Step g of one continuous sequence calls both shapes on copy g mod 64.
    # An untimed pre-roll of 64 steps (every copy once) comes first, then
    # the W warm-up steps, then the K timed steps; so every timed call reads
    # a copy that was last read 64 steps earlier, with the other 63 copies of
    # both shapes (750 MB, three times the Infinity Cache) read in between.
    def step(g: int) -> None:
        call_raw(0, g % copies)
        call_raw(1, g % copies)

    warmup = max(args.warmup, 1)
    preroll = capture(step, copies)
    warm = capture(lambda i: step(copies + i), warmup)
    timed = capture(lambda i: step(copies + warmup + i), args.steps)

    def settle() -> None:
        # The GPU leaves its idle clock only under sustained load (a 20-step
        # timed region alone runs ~0.15 ms, at whatever clock the idle GPU is
        # in): ~0.25 s of pre-roll replays (whole rotations, so the copy
        # order is unchanged) before each timed sequence.
        settle_start = time.perf_counter()
        while time.perf_counter() - settle_start < SETTLE_SECONDS:
            for _ in range(20):
                preroll.replay()
            torch.cuda.synchronize()

    # The K timed steps are enqueued as eager calls, the way the op is called,
    # while untimed pre-roll replays still keep the GPU busy, so every timed
    # kernel is queued before the GPU reaches it and the events bracket the
    # 2K kernels alone. (Replayed as one graph, the same steps carry the
    # graph launch's own 9-10 us of GPU time per replay: reported beside it
    # as value_graph_replay.) Enough pre-roll replays are queued to cover the
    # host's enqueueing of the K steps; if the GPU nevertheless reached the
    # start event before the last timed call was enqueued, the sequence runs
    # again with twice the pre-roll (then falls back to the graph replay).
    settle()
    t0 = time.perf_counter()
    for i in range(8):
        step(copies + warmup + i)
    host_step_s = (time.perf_counter() - t0) / 8
    torch.cuda.synchronize()
    preroll_s = time_graph(preroll)
    rolls = 1 + int(1.5 * args.steps * host_step_s / preroll_s)
    start_ev = torch.cuda.Event(enable_timing=True)
    end_ev = torch.cuda.Event(enable_timing=True)
    timed_launch = None
    for _attempt in range(4):
        settle()
        for _ in range(rolls):
            preroll.replay()
        warm.replay()
        with trace_range("w4a16_fused headline timed steps"):
            start_ev.record()
            for i in range(args.steps):
                step(copies + warmup + i)
            queued = not start_ev.query()
            end_ev.record()
            end_ev.synchronize()
        if queued:
            timed_launch = (f"eager calls, enqueued behind {rolls} untimed pre-roll replays and the warm-up "
                            "(the GPU had not reached the timed region when the last timed call was enqueued)")
            break
        rolls *= 2
    eager_elapsed = start_ev.elapsed_time(end_ev) / 1e3
    if args.headline_pass:
        torch.cuda.synchronize()
        print(json.dumps({"headline_pass": True, "steps": args.steps, "queued": timed_launch is not None,
                          "ms_per_step": round(eager_elapsed / args.steps * 1e3, 5),
                          "us_per_launch": round(eager_elapsed / args.steps / 2 * 1e6, 3),
                          "kernels": [_kernel_name(_lib.plan_linear(xs[j].data_ptr(), layers[j][0][0].data_ptr(),
                                                                    1, n, k), 1, k)
                                      for j, (k, n) in enumerate(shapes)]}), flush=True)
        return 0
    # the same steps as one graph replay, queued behind the pre-roll and warm-up
    settle()
    preroll.replay()
    warm.replay()
    start_ev.record()
    timed.replay()
    end_ev.record()
    end_ev.synchronize()
    graph_elapsed = start_ev.elapsed_time(end_ev) / 1e3
    if timed_launch is None:
        timed_launch = "one graph replay queued behind the pre-roll and warm-up (the eager enqueue could not stay ahead)"
        elapsed = graph_elapsed
    else:
        elapsed = eager_elapsed
    step_bytes = sum(payload_bytes(1, n, k) for k, n in shapes)
    value = step_bytes * args.steps / elapsed / 1e9
    value_graph = step_bytes * args.steps / graph_elapsed / 1e9

    # ---- per-layer and the dominant kernel's roofline ----
    copy_gbps = round(copy_bandwidth(device), 1)
    layer_rows = {}
    for j, (k, n) in enumerate(shapes):
        us = per_layer(lambda i, j=j: call_raw(j, i), copies)
        plan = _lib.plan_linear(xs[j].data_ptr(), layers[j][0][0].data_ptr(), 1, n, k)
        layer_rows[f"K{k}xN{n}"] = {**row_metrics(1, n, k, us, copy_gbps), "kernel": plan,
                                    "kernel_name": _kernel_name(plan, 1, k)}
    # torch-op path (drop-in API) for the same shapes, graph-timed, and its
    # single-call eager latency (launch and Python dispatch included)
    op_us = {f"K{k}xN{n}": round(per_layer(lambda i, j=j: call(j, i), copies), 3) for j, (k, n) in enumerate(shapes)}
    op_eager_us = {f"K{k}xN{n}": round(eager_us(lambda i, j=j: call(j, i), copies), 3)
                   for j, (k, n) in enumerate(shapes)}

    achieved = step_bytes / (elapsed / args.steps) / 1e9  # = value; per-launch average over the two shapes
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBPS, 4),
        "traffic": MEASURED_TRAFFIC_BYTES,
        "traffic_source": TRAFFIC_SOURCE,
        "kernel": " + ".join(r["kernel_name"] for r in layer_rows.values()),
        "bytes_per_launch": step_bytes // 2,
        "us_per_launch": round(elapsed / args.steps / 2 * 1e6, 3),
        "frac_trace": round(step_bytes / 2 / (TRACE_US_PER_LAUNCH * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "trace_us_per_launch": TRACE_US_PER_LAUNCH,
        "trace_source": TRACE_SOURCE,
        "profiler_offset_us": round(TRACE_US_PER_LAUNCH - elapsed / args.steps / 2 * 1e6, 3),
    }

    line = {
        "metric": "INT4 GEMV µs & % of HBM peak per layer (M=1); decode tok/s, 1.1B Llama",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes x f16 -> f32 accumulate",
        "data": "synthetic (weights ~N(0,0.02) fp32 RTN-quantized to INT4 g128, activations ~N(0,1) fp16)",
        "config": {
            "workload": "configs[1]: M=1 MLP layers K2048xN5632 + K5632xN2048, group 128, 64 rotated copies each",
            "step": "one call of each shape (the C-ABI entry point); step g reads copy g mod 64",
            "timed_launch": timed_launch,
            "rotation": f"{SETTLE_SECONDS} s of untimed pre-roll replays (GPU clock settle), then untimed 64-step pre-rolls, then the warm-up steps, then the timed steps, all one "
                        "sequence: every timed call reads a copy last read 64 steps (762 MB of weights) earlier; "
                        f"the timed steps read copies {(copies + warmup) % copies}.. of 64",
            "timed_copies": min(args.steps, copies),
            "parallelism": "single GPU",
        },
        "value_graph_replay": round(value_graph, 1),
        "ms_per_step_graph_replay": round(graph_elapsed / args.steps * 1e3, 5),
        "layers_us": layer_rows,
        "torch_op_us": op_us,
        "torch_op_eager_us": op_eager_us,
        "roofline": roofline,
    }
    line["gpu_state"] = gpu_state_under_load(preroll)
    line["copy_GBps"] = copy_gbps
    if args.profiler == "torch":
        traces = []
        for j, (k, n) in enumerate(shapes):
            path = os.path.join(args.trace_dir, f"torch_fused_M1_K{k}xN{n}.json")
            with trace_range(f"w4a16_fused torch trace K{k}xN{n}"):
                torch_trace(lambda i, j=j: call(j, i), 20, path)
            traces.append(path)
        line["torch_traces"] = traces
    if not args.no_tables:
        line["layers"] = layer_tables(device, copy_gbps)
    if not args.no_decode:
        del layers
        torch.cuda.empty_cache()
        with trace_range("decode configs[4]"):
            line["decode"] = decode_tok_s(device)
        if args.long:
            with trace_range("long prompts and long-context decode"):
                line["decode"].update(prefill_long(device))
                line["decode"].update(decode_long_context(device))
    if not args.no_cpu:
        with trace_range("cpu baseline"):
            line["cpu_baseline"] = cpu_baseline(shapes)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
