"""Benchmark of the fused layer kernels on one MI355X.

One *step* is one pass of the prefill-scale hot path at 4 x 2048 tokens, the
shapes of BASELINE.json configs 4 and 5:

  4a add_rms_norm   residual/hidden [8192, 2560]            -> total, normed
  4b prefill_qkv    packed qkv [8192, 6144], q/k norm + RoPE -> Q, K/V cache
  5a silu_mul       gate_up [8192, 19456]                    -> [8192, 9728]
  5b embedding      8192 ids into [151936, 2560]             -> [8192, 2560]

``value`` is the step's algorithmic HBM bytes (each input read once, each
output written once) divided by its wall time, inputs resident in HBM.  Each
kernel cycles through enough buffer sets that its distinct footprint exceeds
twice the 256 MB Infinity Cache, so repeated calls cannot be served from it.
The step is replayed from captured HIP graphs (as the engine replays its
captured prefill), so host launch overhead is not part of the GPU timeline.
Per-kernel durations come from HIP events around graphs of GRAPH_CALLS (96)
back-to-back launches of one kernel (rotating its buffer sets), divided by
96: long enough that the graph's own launch cost adds under 0.1 us per call,
so the figure matches the kernel trace's average duration.  Decode
configs 1-3 are timed the same way (microseconds per call), and so are the
split-K decode projections of one Qwen3-4B layer at batch 1-64, beside the
F.linear (hipBLASLt) path they replace, decode attention at the engine
contract's public workloads beside torch's scaled_dot_product_attention, and
the causal prefill attention beside torch's flash kernel.  The CPU baseline
(``cpu_baseline``) is the whole step through the reference's PyTorch formulas
on the host CPU (up to 16 threads, CPU model stated); ``cpu_reference`` also
times every BASELINE config that way, and ``cpu_baseline_oracle`` is the C
oracle (one thread) on the step's shapes.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from collections import deque
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from starter_amd.kernels.decode_fused import add_rms_norm, qkv_norm_rope_cache, silu_mul  # noqa: E402
from starter_amd.kernels.embedding import embedding  # noqa: E402
from starter_amd.kernels.prefill import prefill_qkv  # noqa: E402
from starter_amd.kernels.qk_norm_rope import qk_norm_rope  # noqa: E402
from starter_amd.kernels.rmsnorm import rms_norm  # noqa: E402
from starter_amd.kernels.rotary import default_inv_freq, rope_tables  # noqa: E402
from starter_amd.kernels import lm_head as _lm_head, row_gemv, skinny_gemm  # noqa: E402
from starter_amd.kernels.small_query_attention import SmallQueryAttention  # noqa: E402
from starter_amd.engine import KEY_ALIGN  # noqa: E402

METRIC = ("achieved HBM GB/s (% of MI355X peak) + µs/call per fused kernel, decode & prefill")
PEAK_GBPS = 8000.0          # MI355X HBM3E, AMD specification
INFINITY_CACHE = 256 << 20  # bytes
H, I, V = 2560, 9728, 151936
NQ, NK, D = 32, 8, 128
B, T = 4, 2048
TOKENS = B * T
CAPACITY = T + 128
BF16 = torch.bfloat16


def bf16_bytes(*numels: int) -> int:
    return 2 * sum(numels)


# Algorithmic bytes per call (each input once, each output once, gains and tables).
BYTES = {
    "add_rms_norm": bf16_bytes(4 * TOKENS * H, H),
    "prefill_qkv": bf16_bytes(2 * TOKENS * (NQ + 2 * NK) * D, 2 * D, 2 * T * D),
    "silu_mul": bf16_bytes(3 * TOKENS * I),
    "embedding": bf16_bytes(2 * TOKENS * H) + 8 * TOKENS,
}
ROWS = {"add_rms_norm": TOKENS, "prefill_qkv": TOKENS * (NQ + 2 * NK), "silu_mul": TOKENS,
        "embedding": TOKENS}
ROW_UNIT = {"add_rms_norm": "rows", "prefill_qkv": "head-rows", "silu_mul": "rows",
            "embedding": "tokens"}


def normal(shape, mean=0.0, std=1.0, g=None, device="cuda"):
    t = torch.empty(shape, dtype=torch.float32, device=device)
    t.normal_(mean, std, generator=g)
    return t.to(BF16)


def sets_for(footprint: int) -> int:
    """Buffer sets needed so the rotation's footprint exceeds 2x the Infinity Cache."""
    return max(2, -(-2 * INFINITY_CACHE // footprint) + 1)


class Workload:
    """Device buffers of the prefill step, several rotating sets per kernel."""

    def __init__(self, device):
        g = torch.Generator(device=device).manual_seed(0)
        self.w = normal((H,), 1.0, 0.1, g)
        self.qw, self.kw = normal((D,), 1.0, 0.1, g), normal((D,), 1.0, 0.1, g)
        self.cos, self.sin = rope_tables(default_inv_freq(5_000_000, D), CAPACITY, device=device)
        n = sets_for(BYTES["add_rms_norm"])
        self.add = [(normal((TOKENS, H), g=g), normal((TOKENS, H), g=g)) for _ in range(n)]
        n = sets_for(BYTES["prefill_qkv"])
        self.qkv = [(normal((TOKENS, (NQ + 2 * NK) * D), g=g),
                     torch.zeros((B, NK, CAPACITY, D), dtype=BF16, device=device),
                     torch.zeros((B, NK, CAPACITY, D), dtype=BF16, device=device))
                    for _ in range(n)]
        n = sets_for(BYTES["silu_mul"])
        self.gate_up = [normal((TOKENS, 2 * I), g=g) for _ in range(n)]
        self.table = normal((V, H), 0.0, 0.02, g)
        n = sets_for(BYTES["embedding"])
        self.ids = [torch.randint(0, V, (TOKENS,), generator=g, device=device) for _ in range(n)]
        self.sets = {"add_rms_norm": len(self.add), "prefill_qkv": len(self.qkv),
                     "silu_mul": len(self.gate_up), "embedding": len(self.ids)}
        # The wrappers allocate fresh outputs; keeping the last `sets` of them
        # alive makes the caching allocator rotate output buffers too.
        self.live = {name: deque(maxlen=n) for name, n in self.sets.items()}

    def launch(self, name: str, k: int):
        if name == "add_rms_norm":
            r, h = self.add[k % len(self.add)]
            out = add_rms_norm(r, h, self.w, 1e-6)
        elif name == "prefill_qkv":
            qkv, kc, vc = self.qkv[k % len(self.qkv)]
            out = prefill_qkv(qkv, self.qw, self.kw, 1e-6, 1e-6, self.cos, self.sin, kc, vc, T)
        elif name == "silu_mul":
            out = silu_mul(self.gate_up[k % len(self.gate_up)])
        else:
            out = embedding(self.ids[k % len(self.ids)], self.table)
        self.live[name].append(out)


KERNELS = ("embedding", "add_rms_norm", "prefill_qkv", "silu_mul")
GRAPH_CALLS = 96  # launches per timing graph
STEPS_PER_GRAPH = 8  # one captured graph holds this many consecutive steps


def capture(fn):
    """Capture ``fn``'s launches into a HIP graph (after warmups on the capture stream)."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    torch.cuda.synchronize()
    return graph


def timed_replays(graph, replays: int) -> list[float]:
    """Microseconds of each replay, from HIP events on the replay stream."""
    samples = []
    for _ in range(replays):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end) * 1e3)
    return samples


def kernel_durations(work: Workload, calls: int, replays: int) -> dict:
    """Per-kernel microseconds per call: one graph per kernel of ``calls``
    back-to-back launches rotating its buffer sets; the graphs are replayed
    round-robin ``replays`` times (after a warm-up) so clock or thermal drift
    affects every kernel alike.  Returns every replay's per-call average."""
    graphs = {name: capture(lambda name=name: [work.launch(name, k) for k in range(calls)])
              for name in KERNELS}
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.5:  # bring clocks to their steady state
        for graph in graphs.values():
            graph.replay()
        torch.cuda.synchronize()
    out = {name: [] for name in KERNELS}
    for _ in range(replays):
        for name, graph in graphs.items():
            out[name].append(timed_replays(graph, 1)[0] / calls)
    del graphs
    return out


def run_prefill_step(work: Workload, steps: int, warmup: int):
    """Wall time of exactly ``steps`` steps, replayed from graphs of
    STEPS_PER_GRAPH consecutive steps (plus one graph for the remainder)."""
    def steps_fn(first, count):
        def fn():
            for k in range(first, first + count):
                for name in KERNELS:
                    work.launch(name, k)
        return fn

    full, rest = divmod(steps, STEPS_PER_GRAPH)
    graph = capture(steps_fn(0, STEPS_PER_GRAPH))
    tail = capture(steps_fn(0, rest)) if rest else None
    for _ in range(max(1, -(-warmup // STEPS_PER_GRAPH))):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(full):
        graph.replay()
    if tail is not None:
        tail.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) * 1e-3


def graph_time(fn, calls_per_replay: int, replays: int = 50) -> float:
    """Median microseconds per call of ``fn`` captured ``calls_per_replay`` times in one graph."""
    graph = capture(lambda: [fn() for _ in range(calls_per_replay)])
    for _ in range(5):
        graph.replay()
    torch.cuda.synchronize()
    return statistics.median(t / calls_per_replay for t in timed_replays(graph, replays))


def decode_configs(device) -> dict:
    g = torch.Generator(device=device).manual_seed(0)
    out = {}
    # Config 1: RMSNorm [8, 2560].
    x, w = normal((8, H), g=g), normal((H,), 1.0, 0.1, g)
    us = graph_time(lambda: rms_norm(x, w, 1e-6), 100)
    out["config1_rms_norm_8x2560"] = {"us_per_call": us, "bytes": bf16_bytes(2 * 8 * H, H),
                                      "rows": 8}
    # Config 2: add + RMSNorm [64, 2560] chained over 36 layers.
    residual = normal((64, H), 0.0, 4.0, g)
    hidden = normal((36, 64, H), g=g)
    ws = normal((36, H), 1.0, 0.1, g)

    def layers():
        r = residual
        for layer in range(36):
            r, _ = add_rms_norm(r, hidden[layer], ws[layer], 1e-6)
        return r

    us = graph_time(layers, 1) / 36
    out["config2_add_rms_norm_64x2560_x36"] = {"us_per_call": us,
                                               "bytes": bf16_bytes(4 * 64 * H, H), "rows": 64}
    # Config 3: QK-norm + RoPE, 32 sequences, per-sequence positions in [0, 32767].
    q, k = normal((32, 32, 1, D), g=g), normal((32, 8, 1, D), g=g)
    qw, kw = normal((D,), 1.0, 0.1, g), normal((D,), 1.0, 0.1, g)
    positions = torch.randint(0, 32768, (32,), generator=g, device=device)
    cos, sin = rope_tables(default_inv_freq(5_000_000, D), positions=positions)
    cos, sin = cos.view(32, 1, D), sin.view(32, 1, D)
    us = graph_time(lambda: qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6, 1e-6), 100)
    out["config3_qk_norm_rope_b32"] = {"us_per_call": us,
                                       "bytes": bf16_bytes(2 * 32 * 40 * D, 2 * D, 2 * 32 * D),
                                       "rows": 32 * 40}
    # The other fused kernels at decode batch 64 (the north star's < 5 us/call
    # bound applies to every fused kernel at batch <= 64).
    gate_up = normal((64, 2 * I), g=g)
    us = graph_time(lambda: silu_mul(gate_up), 100)
    out["decode_silu_mul_64x9728"] = {"us_per_call": us, "bytes": bf16_bytes(3 * 64 * I),
                                      "rows": 64}
    table = normal((V, H), 0.0, 0.02, g)
    ids = torch.randint(0, V, (64,), generator=g, device=device)
    us = graph_time(lambda: embedding(ids, table), 100)
    out["decode_embedding_64_ids"] = {"us_per_call": us, "bytes": bf16_bytes(2 * 64 * H) + 8 * 64,
                                      "rows": 64}
    del table
    qkv = normal((64, (NQ + 2 * NK) * D), g=g)
    kc = torch.zeros((64, NK, CAPACITY, D), dtype=BF16, device=device)
    vc = torch.zeros_like(kc)
    ctab, stab = rope_tables(default_inv_freq(5_000_000, D), CAPACITY, device=device)
    pos = torch.tensor([T], device=device)
    us = graph_time(lambda: qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 1e-6, ctab, stab, pos, kc, vc), 100)
    out["decode_qkv_norm_rope_cache_b64"] = {
        "us_per_call": us, "rows": 64 * (NQ + 2 * NK),
        "bytes": bf16_bytes(64 * (NQ + 2 * NK) * D + 64 * (NQ + 2 * NK) * D, 2 * D, 2 * D) + 8}
    for entry in out.values():
        entry["rows_per_s"] = entry["rows"] / (entry["us_per_call"] * 1e-6)
        entry["gbps"] = entry["bytes"] / (entry["us_per_call"] * 1e3)
        entry["frac"] = entry["gbps"] / PEAK_GBPS
        entry["under_5us"] = entry["us_per_call"] < 5.0
    return out


#: Decode projections of one Qwen3-4B layer: (n, k) of W [n, k]; gate_up is packed [2n, k].
PROJECTIONS = {"qkv": (6144, 2560), "o_proj": (H, 4096), "gate_up": (I, H), "down": (H, I)}
PROJECTION_ROWS = (1, 4, 16, 64)


def decode_projections(device, replays: int = 20, calls: int = GRAPH_CALLS) -> dict:
    """Split-K projections (linear_partials / linear_silu_mul) at decode batch
    1-64 on the Qwen3-4B layer shapes, next to the unfused path the engine
    takes without them (F.linear on hipBLASLt, plus silu_mul for gate/up),
    and at batch 1 the one-workgroup-per-CU forms the engine runs there
    (row_gemv, with the add or norm of the neighbouring add + norm folded in).
    Weights rotate over enough copies to exceed twice the Infinity Cache, as
    in decode, where 36 layers of weights (7.3 GB) stream from HBM each step."""
    g = torch.Generator(device=device).manual_seed(1)
    out = {}
    for name, (n, k) in PROJECTIONS.items():
        rows_w = 2 * n if name == "gate_up" else n
        w_bytes = bf16_bytes(rows_w * k)
        weights = [normal((rows_w, k), 0.0, k ** -0.5, g) for _ in range(sets_for(w_bytes))]
        entry = {}
        for m in PROJECTION_ROWS:
            x = normal((m, k), g=g)
            if name == "gate_up":
                ours = lambda i, x=x: skinny_gemm.linear_silu_mul(x, weights[i % len(weights)])
                base = lambda i, x=x: silu_mul(torch.nn.functional.linear(x, weights[i % len(weights)]))
                out_bytes, splits = bf16_bytes(m * n), 1
            else:
                ours = lambda i, x=x: skinny_gemm.linear_partials(x, weights[i % len(weights)])
                base = lambda i, x=x: torch.nn.functional.linear(x, weights[i % len(weights)])
                splits = skinny_gemm.split_count(n, k, m)
                out_bytes = 4 * splits * m * n
            t_ours = graph_time_rotating(ours, calls, replays)
            t_base = graph_time_rotating(base, calls, replays)
            moved = w_bytes + bf16_bytes(m * k) + out_bytes
            entry[f"m{m}"] = {"us_per_call": t_ours, "bytes": moved, "splits": splits,
                              "gbps": moved / (t_ours * 1e3), "frac": moved / (t_ours * 1e3) / PEAK_GBPS,
                              "hipblaslt_us": t_base, "speedup_vs_hipblaslt": t_base / t_ours}
            print(f"bench: proj {name:8s} m={m:2d} {t_ours:7.2f} us ({100 * entry[f'm{m}']['frac']:.1f}% "
                  f"of peak)  F.linear path {t_base:7.2f} us", file=sys.stderr, flush=True)
        # The engine's batch-1 form: whole-K workgroups, one per CU, with the
        # residual add (o_proj, down) or the RMSNorm (qkv; gate/up with SiLU)
        # folded in (no add + norm launch between projections).
        x = normal((1, k), g=g)
        sq = torch.ones((1, row_gemv.GROUPS), dtype=torch.float64, device=device)
        gain = normal((k,), 1.0, 0.1, g)
        if name == "gate_up":
            fold = lambda i: row_gemv.linear_silu_mul_normed(x, sq, gain, 1e-6, weights[i % len(weights)])
            kind, out_bytes = "norm prologue + SiLU*up", bf16_bytes(n)
        elif name == "qkv":
            fold = lambda i: row_gemv.linear_normed(x, sq, gain, 1e-6, weights[i % len(weights)])
            kind, out_bytes = "norm prologue", bf16_bytes(n)
        else:
            residual = normal((1, n), g=g)
            fold = lambda i: row_gemv.linear_residual(x, weights[i % len(weights)], residual)
            kind, out_bytes = "residual epilogue", bf16_bytes(2 * n) + 8 * row_gemv.GROUPS
        t_fold = graph_time_rotating(fold, calls, replays)
        moved = w_bytes + bf16_bytes(k) + out_bytes
        entry["m1_folded"] = {"us_per_call": t_fold, "bytes": moved, "kind": kind,
                              "gbps": moved / (t_fold * 1e3), "frac": moved / (t_fold * 1e3) / PEAK_GBPS}
        print(f"bench: proj {name:8s} m= 1 {t_fold:7.2f} us ({100 * entry['m1_folded']['frac']:.1f}% "
              f"of peak)  one workgroup per CU, {kind}", file=sys.stderr, flush=True)
        out[name] = entry
        del weights
        torch.cuda.empty_cache()
    for m in PROJECTION_ROWS:
        ours = sum(out[name][f"m{m}"]["us_per_call"] for name in PROJECTIONS)
        base = sum(out[name][f"m{m}"]["hipblaslt_us"] for name in PROJECTIONS)
        out[f"layer_m{m}"] = {"us": ours, "hipblaslt_us": base, "speedup_vs_hipblaslt": base / ours}
    return out


#: Decode attention of the contract's public workloads (batch, prompt + output
#: tokens + 1): every used key of every layer is read once per step.
ATTENTION_CASES = ((1, 545), (4, 2081), (16, 641))


def decode_attention_bench(device, replays: int = 20, calls: int = GRAPH_CALLS) -> dict:
    """SmallQueryAttention.run at full cache length on the Qwen3-4B head
    layout (32 query heads, 8 KV heads, width 128), K/V rotating over copies
    beyond twice the Infinity Cache; beside torch's scaled_dot_product_attention
    with GQA on the same tensors (the engine's other GPU path is torch's own
    flash attention)."""
    g = torch.Generator(device=device).manual_seed(2)
    out = {}
    for batch, cap in ATTENTION_CASES:
        kv_bytes = bf16_bytes(2 * batch * NK * cap * D)
        sets = sets_for(kv_bytes)
        caches = [(normal((batch, NK, cap, D), g=g), normal((batch, NK, cap, D), g=g)) for _ in range(sets)]
        q = normal((batch, NQ, 1, D), g=g)
        used = torch.full((batch * NK,), cap, dtype=torch.int32, device=device)
        plan = SmallQueryAttention(batch, NQ, NK, cap, device, key_align=KEY_ALIGN)
        ours = lambda i: plan.run(q, *caches[i % sets], used, D ** -0.5)
        base = lambda i: torch.nn.functional.scaled_dot_product_attention(
            q, *caches[i % sets], scale=D ** -0.5, enable_gqa=True)
        t_ours = graph_time_rotating(ours, calls, replays)
        try:
            t_base = graph_time_rotating(base, calls, replays)
        except RuntimeError:
            t_base = None
        moved = kv_bytes + bf16_bytes(2 * batch * NQ * D)
        key = f"b{batch}_ctx{cap}"
        out[key] = {"us_per_call": t_ours, "bytes": moved, "splits": plan.splits,
                    "gbps": moved / (t_ours * 1e3), "frac": moved / (t_ours * 1e3) / PEAK_GBPS,
                    "torch_sdpa_us": t_base}
        print(f"bench: attention {key:12s} {t_ours:7.2f} us ({100 * out[key]['frac']:.1f}% of peak, "
              f"{plan.splits} splits)  torch sdpa {t_base if t_base is None else round(t_base, 2)} us",
              file=sys.stderr, flush=True)
        del caches
        torch.cuda.empty_cache()
    return out


#: Causal prefill attention at the Qwen3-4B heads (batch, prompt tokens).
PREFILL_ATTENTION_CASES = ((4, 2048), (1, 4096), (16, 512))
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 matrix peak, AMD specification


def prefill_attention_bench(device, replays: int = 20, calls: int = 8) -> dict:
    """``prefill_attention`` (qf_prefill_attention) on the prompt's own cache
    slots, beside torch's flash kernel on the same tensors (the reference's
    prefill attention, engine/prefill.py:13-23).  Matrix-core bound: the
    figure is causal flops (4 * B * Hq * T(T+1)/2 * 128) per second against
    the dense bf16 peak."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from starter_amd.kernels.prefill import prefill_attention
    g = torch.Generator(device=device).manual_seed(3)
    out = {}
    for batch, length in PREFILL_ATTENTION_CASES:
        q = normal((batch, length, NQ, D), g=g)
        keys = normal((batch, NK, length + 32, D), g=g)
        values = normal((batch, NK, length + 32, D), g=g)
        scale = D ** -0.5
        flops = 4.0 * batch * NQ * (length * (length + 1) / 2) * D
        t_ours = graph_time(lambda: prefill_attention(q, keys, values, length, scale), calls, replays)

        def flash():
            with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                return torch.nn.functional.scaled_dot_product_attention(
                    q.transpose(1, 2), keys[:, :, :length], values[:, :, :length], is_causal=True,
                    scale=scale, enable_gqa=True)
        try:
            t_flash = graph_time(flash, calls, replays)
        except RuntimeError:
            t_flash = None
        tflops = flops / (t_ours * 1e6)
        key = f"b{batch}_t{length}"
        out[key] = {"us_per_call": t_ours, "flops": flops, "tflops": tflops,
                    "frac": tflops / PEAK_BF16_TFLOPS, "torch_flash_us": t_flash}
        print(f"bench: prefill attention {key:10s} {t_ours:8.1f} us ({tflops:6.1f} TFLOP/s, "
              f"{100 * tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)  torch flash "
              f"{t_flash if t_flash is None else round(t_flash, 1)} us", file=sys.stderr, flush=True)
        del q, keys, values
        torch.cuda.empty_cache()
    return out


#: The engine contract's public workloads (batch, prompt tokens, output tokens),
#: plus batch 2 (the largest batch whose decode step folds the add + norm
#: launches into its projections) and batch 64 (the largest batch the split-K
#: decode projections serve).
ENGINE_WORKLOADS = ((1, 512, 32), (2, 512, 32), (4, 2048, 32), (16, 512, 128), (64, 512, 32))


def engine_decode(device, steps: int = 32, workloads=ENGINE_WORKLOADS) -> dict:
    """End to end: starter_amd.engine.Engine on a randomly initialised
    Qwen3-4B (the real architecture: 36 layers, hidden 2560, vocab 151936,
    tied embedding) generating at the public workloads; the decode steps are
    HIP-graph replays.  Reports decode tokens/s and the step's algorithmic
    bytes (every weight once, the LM head, the K/V prefix read and the new
    K/V rows written) against the HBM roofline."""
    from transformers import Qwen3Config
    from starter_amd.engine import Engine
    cfg = Qwen3Config(vocab_size=V, hidden_size=H, intermediate_size=I, num_hidden_layers=36,
                      num_attention_heads=NQ, num_key_value_heads=NK, head_dim=D,
                      max_position_embeddings=40960, rope_theta=1_000_000, rms_norm_eps=1e-6,
                      tie_word_embeddings=True)
    engine = Engine(config=cfg, seed=0, device=device)
    weight_bytes = sum(2 * t.numel() for layer in engine.layers
                       for t in (layer.qkv, layer.o, layer.gate_up, layer.down))
    weight_bytes += 2 * engine.lm_head.numel()
    out = {"model": "Qwen3-4B architecture, random bf16 weights", "weight_bytes": weight_bytes}
    g = torch.Generator().manual_seed(5)
    for batch, length, new in workloads:
        prompts = torch.randint(0, V, (batch, length), generator=g).tolist()
        count = min(new, steps + 1)
        # first call of a shape: state allocation, prefill graph capture and
        # replay, decode graph capture.  next() returns once the first tokens
        # are on the host (the generator waits for them, nothing more).
        gen = engine.generate(prompts, count)
        t0 = time.perf_counter()
        next(gen)
        t_first = time.perf_counter() - t0
        t1 = time.perf_counter()
        done = sum(1 for _ in gen)      # count - 1 decode steps, one host read each
        t_decode = time.perf_counter() - t1
        # later calls of the same shape replay both graphs: warm time to first
        # tokens (prompt upload + prefill replay + token download) and decode
        warm = []
        for _ in range(2):
            gen = engine.generate(prompts, count)
            t0 = time.perf_counter()
            next(gen)
            warm.append(time.perf_counter() - t0)
            t1 = time.perf_counter()
            done = sum(1 for _ in gen)
            t_decode = min(t_decode, time.perf_counter() - t1)
        t_prefill = min(warm)
        step_us = t_decode / done * 1e6
        mid = length + done // 2        # average prefix length over the timed steps
        kv = 36 * batch * NK * mid * D * 2 * 2 + 36 * batch * NK * D * 2 * 2
        step_bytes = weight_bytes + kv + bf16_bytes(batch * H)
        key = f"b{batch}_p{length}"
        # the engine contract's figure for the whole workload (QWEN_ENGINE_CONTRACT.md:88-94):
        # batch x output tokens / (time to the first tokens + the remaining
        # steps), here from the warm first-token time and the measured step
        total_s = t_prefill + (new - 1) * step_us * 1e-6
        out[key] = {"decode_steps": done, "us_per_step": step_us,
                    "tokens_per_s": batch / (step_us * 1e-6),
                    "output_tokens": new, "workload_tokens_per_s": batch * new / total_s,
                    "prefill_ms": t_prefill * 1e3, "prefill_tokens_per_s": batch * length / t_prefill,
                    "first_call_s": t_first,
                    "step_bytes": step_bytes, "gbps": step_bytes / (step_us * 1e3),
                    "frac": step_bytes / (step_us * 1e3) / PEAK_GBPS}
        print(f"bench: engine {key:10s} decode {step_us:8.1f} us/step  {out[key]['tokens_per_s']:8.1f} tok/s "
              f"({100 * out[key]['frac']:.1f}% of HBM roofline)  prefill {t_prefill * 1e3:.2f} ms warm "
              f"({t_first:.2f} s first call, with allocation and capture)  "
              f"{out[key]['workload_tokens_per_s']:.0f} tok/s for {batch} x {new} output tokens",
              file=sys.stderr, flush=True)
    del engine
    torch.cuda.empty_cache()
    return out


def graph_time_rotating(fn, calls: int, replays: int) -> float:
    """Median microseconds per call of ``fn(i)``, i = 0..calls-1, captured in one graph."""
    graph = capture(lambda: [fn(i) for i in range(calls)])
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    return statistics.median(t / calls for t in timed_replays(graph, replays))


def copy_bandwidth(device) -> float:
    """GB/s of a plain 1 GiB device-to-device copy (read + write counted)."""
    src = torch.empty(1 << 29, dtype=BF16, device=device)
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    samples = []
    for _ in range(10):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        dst.copy_(src)
        end.record()
        end.synchronize()
        samples.append(2 * src.numel() * 2 / (start.elapsed_time(end) * 1e6))
    del src, dst
    return statistics.median(samples)


def cpu_baseline(reps: int = 3) -> dict:
    """The C oracle (one thread) on the step's shapes; median of ``reps`` after one warmup."""
    import numpy as np

    from oracle import oracle as O

    rng = np.random.default_rng(0)

    def draw(shape, mean=0.0, std=1.0):
        return O.bf16_bits((rng.standard_normal(shape, dtype=np.float32) * std + mean))

    w = draw((H,), 1.0, 0.1)
    res, hid = draw((TOKENS, H)), draw((TOKENS, H))
    qkv = draw((TOKENS, (NQ + 2 * NK) * D))
    qw, kw = draw((D,), 1.0, 0.1), draw((D,), 1.0, 0.1)
    cos, sin = O.rope_table(O.default_inv_freq(5_000_000, D), n_pos=CAPACITY)
    cache = np.zeros((B, NK, CAPACITY, D), np.uint16)
    gate_up = draw((TOKENS, 2 * I))
    table = draw((V, H), 0.0, 0.02)
    ids = rng.integers(0, V, TOKENS)

    def step():
        O.embedding(ids, table)
        O.add_rms_norm(res, hid, w, 1e-6)
        O.prefill_qkv(qkv, qw, kw, 1e-6, 1e-6, cos, sin, cache, cache, T)
        O.silu_mul(gate_up)

    step()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    seconds = statistics.median(times)
    step_bytes = sum(BYTES.values())
    return {"value": step_bytes / seconds / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"C oracle, whole 4x2048-token step (4 kernels), median of {reps} reps "
                      f"after 1 warmup: {seconds * 1e3:.0f} ms/step",
            "cpu": cpu_model(), "host_cpus": os.cpu_count()}


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def torch_cpu_configs(reps_small: int = 20, reps_large: int = 3) -> dict:
    """Each BASELINE config through the reference's PyTorch formulas on the
    host CPU, bf16 tensors as the engine holds them: Qwen3RMSNorm.forward
    (f32 mean of squares, rsqrt, cast, gain), the residual add, the per-head
    norm + apply_rotary_pos_emb (rotate-half, cos/sin rows of
    Qwen3RotaryEmbedding), F.silu(gate) * up and F.embedding.  Threads: the
    host's cores, at most 16 (one GPU's share of the box).  Median of
    ``reps`` after one warm-up call.  A reported baseline only."""
    from torch.nn import functional as F

    threads = max(1, min(os.cpu_count() or 1, 16))
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)

    def draw(shape, mean=0.0, std=1.0):
        return (torch.randn(shape, generator=g) * std + mean).to(BF16)

    def norm(x, w, eps=1e-6):
        f = x.float()
        f = f * torch.rsqrt(f.pow(2).mean(-1, keepdim=True) + eps)
        return w * f.to(BF16)

    def rotate_half(x):
        return torch.cat((-x[..., D // 2:], x[..., : D // 2]), dim=-1)

    def tables(positions):
        inv = default_inv_freq(5_000_000, D)
        ang = positions.float()[:, None] * inv[None, :]
        emb = torch.cat((ang, ang), dim=-1)
        return emb.cos().to(BF16), emb.sin().to(BF16)

    def timed(fn, reps):
        fn()
        samples = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            samples.append(time.perf_counter() - t0)
        return statistics.median(samples)

    out = {}

    def record(name, seconds, rows, bytes_):
        out[name] = {"us_per_call": seconds * 1e6, "rows_per_s": rows / seconds,
                     "gbps": bytes_ / seconds / 1e9}

    with torch.inference_mode():
        x, w = draw((8, H)), draw((H,), 1.0, 0.1)
        record("config1_rms_norm_8x2560", timed(lambda: norm(x, w), reps_small), 8,
               bf16_bytes(2 * 8 * H, H))

        residual, hidden, ws = draw((64, H), 0.0, 4.0), draw((36, 64, H)), draw((36, H), 1.0, 0.1)

        def layers():
            r = residual
            for layer in range(36):
                r = r + hidden[layer]
                norm(r, ws[layer])

        record("config2_add_rms_norm_64x2560_x36", timed(layers, reps_small) / 36, 64,
               bf16_bytes(4 * 64 * H, H))

        q, k = draw((32, 1, NQ, D)), draw((32, 1, NK, D))
        qw, kw = draw((D,), 1.0, 0.1), draw((D,), 1.0, 0.1)
        cos3, sin3 = tables(torch.randint(0, 32768, (32,), generator=g))
        cos3, sin3 = cos3.view(32, 1, 1, D), sin3.view(32, 1, 1, D)

        def qk_rope(q, k, cos, sin):
            qn = norm(q.transpose(1, 2), qw)
            kn = norm(k.transpose(1, 2), kw)
            return qn * cos + rotate_half(qn) * sin, kn * cos + rotate_half(kn) * sin

        record("config3_qk_norm_rope_b32", timed(lambda: qk_rope(q, k, cos3, sin3), reps_small),
               32 * (NQ + NK), bf16_bytes(2 * 32 * (NQ + NK) * D, 2 * D, 2 * 32 * D))

        res4, hid4, w4 = draw((TOKENS, H)), draw((TOKENS, H)), draw((H,), 1.0, 0.1)

        def add_norm():
            total = res4 + hid4
            return total, norm(total, w4)

        record("config4a_add_rms_norm_8192x2560", timed(add_norm, reps_large), TOKENS,
               BYTES["add_rms_norm"])

        # Config 4b as the GPU leg runs it (prefill_qkv at the engine's call
        # site, engine/prefill.py:39-43): the packed Q|K|V rows' per-head
        # norm + RoPE, K written into the cache, V copied into it.
        cos4, sin4 = tables(torch.arange(T))
        cos4, sin4 = cos4.view(1, 1, T, D), sin4.view(1, 1, T, D)
        qkv4 = draw((TOKENS, (NQ + 2 * NK) * D))
        keys4 = torch.zeros((B, NK, CAPACITY, D), dtype=BF16)
        values4 = torch.zeros_like(keys4)

        def packed_qkv():
            heads = qkv4.view(B, T, NQ + 2 * NK, D).transpose(1, 2)      # [B, H, T, D]
            qn, kn = norm(heads[:, :NQ], qw), norm(heads[:, NQ:NQ + NK], kw)
            q = qn * cos4 + rotate_half(qn) * sin4
            keys4[:, :, :T] = kn * cos4 + rotate_half(kn) * sin4
            values4[:, :, :T] = heads[:, NQ + NK:]
            return q

        record("config4b_prefill_qkv_4x2048", timed(packed_qkv, reps_large), TOKENS * (NQ + 2 * NK),
               BYTES["prefill_qkv"])
        del res4, hid4, qkv4, keys4, values4

        gate_up = draw((TOKENS, 2 * I))
        record("config5a_silu_mul_8192x9728",
               timed(lambda: F.silu(gate_up[:, :I]) * gate_up[:, I:], reps_large), TOKENS,
               BYTES["silu_mul"])
        del gate_up

        table = draw((V, H), 0.0, 0.02)
        ids = torch.randint(0, V, (TOKENS,), generator=g)
        record("config5b_embedding_8192_ids", timed(lambda: F.embedding(ids, table), reps_large),
               TOKENS, BYTES["embedding"])

        # The GPU step's four calls on its shapes: gather, add + norm, the
        # packed Q|K|V row's head norm + RoPE with the K and V cache fill
        # (engine/prefill.py:34-51), SiLU * up.
        res4, hid4 = draw((TOKENS, H)), draw((TOKENS, H))
        qkv = draw((TOKENS, (NQ + 2 * NK) * D))
        keys = torch.zeros((B, NK, CAPACITY, D), dtype=BF16)
        values = torch.zeros_like(keys)
        gate_up = draw((TOKENS, 2 * I))

        def step():
            F.embedding(ids, table)
            total = res4 + hid4
            norm(total, w4)
            heads = qkv.view(B, T, NQ + 2 * NK, D).transpose(1, 2)      # [B, H, T, D]
            qn, kn = norm(heads[:, :NQ], qw), norm(heads[:, NQ:NQ + NK], kw)
            q = qn * cos4 + rotate_half(qn) * sin4
            keys[:, :, :T] = kn * cos4 + rotate_half(kn) * sin4
            values[:, :, :T] = heads[:, NQ + NK:]
            F.silu(gate_up[:, :I]) * gate_up[:, I:]
            return q

        step_s = timed(step, reps_large)
        del table, gate_up, qkv, keys, values, res4, hid4
    torch.set_num_threads(previous)
    step_bytes = sum(BYTES.values())
    return {"threads": threads, "cpu": cpu_model(), "host_cpus": os.cpu_count(),
            "what": "reference PyTorch formulas on the host CPU (bf16 tensors)", "configs": out,
            "step": {"seconds": step_s, "bytes": step_bytes, "gbps": step_bytes / step_s / 1e9,
                     "reps": reps_large}}


CALIBRATION_BYTES = 256 << 20  # one-way size of the --profile calibration copy
PMC_SUMMARY = ROOT / "profiles" / "pmc_prefill_kernels.json"


def pmc_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of ``kernel`` measured by rocprofv3 FETCH_SIZE and
    WRITE_SIZE (committed summary, written from a ``--profile`` run)."""
    if not PMC_SUMMARY.exists():
        return None
    entry = json.loads(PMC_SUMMARY.read_text()).get("kernels", {}).get(kernel)
    return None if entry is None else entry["hbm_bytes_per_launch"]


def profile_run(device, launches: int) -> None:
    """Eager launches for counter collection: a calibration copy of known size
    (CALIBRATION_BYTES read + written by torch's copy kernel), then each
    prefill kernel ``launches`` times on rotating buffer sets, then each decode
    projection and the LM head at batch 1, 16 and 64 ``launches`` times on
    rotating weights, then the prefill attention at 4 x 2048."""
    src = torch.empty(CALIBRATION_BYTES // 2, dtype=BF16, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    work = Workload(device)
    torch.cuda.synchronize()
    for name in KERNELS:
        for k in range(launches):
            work.launch(name, k)
        torch.cuda.synchronize()
    del work
    torch.cuda.empty_cache()
    # Decode projections at batch 1, 16 and 64, in this order (dispatch order
    # tells apart projections that share a kernel instantiation).
    g = torch.Generator(device=device).manual_seed(1)
    order = []
    for name, (n, k) in PROJECTIONS.items():
        rows_w = 2 * n if name == "gate_up" else n
        weights = [normal((rows_w, k), 0.0, k ** -0.5, g) for _ in range(sets_for(bf16_bytes(rows_w * k)))]
        for m in (1, 16, 64):
            x = normal((m, k), g=g)
            fn = skinny_gemm.linear_silu_mul if name == "gate_up" else skinny_gemm.linear_partials
            for i in range(launches):
                fn(x, weights[i % len(weights)])
            torch.cuda.synchronize()
            order.append(f"{name}_m{m}")
        del weights
        torch.cuda.empty_cache()
    # The LM head with the greedy choice over the Qwen3-4B vocabulary at the
    # same batches (projection kernel, then the candidate reduction).
    heads = [normal((V, H), 0.0, 0.02, g) for _ in range(sets_for(bf16_bytes(V * H)))]
    for m in (1, 16, 64):
        x = normal((m, H), g=g)
        for i in range(launches):
            _lm_head.lm_head_argmax(x, heads[i % len(heads)])
        torch.cuda.synchronize()
        order.append(f"lm_head_m{m}")
    del heads
    torch.cuda.empty_cache()
    # The causal prefill attention at 4 x 2048 (the first of its bench cases).
    from starter_amd.kernels.prefill import prefill_attention
    batch, length = PREFILL_ATTENTION_CASES[0]
    q = normal((batch, length, NQ, D), g=g)
    keys = normal((batch, NK, length + 32, D), g=g)
    values = normal((batch, NK, length + 32, D), g=g)
    for _ in range(launches):
        prefill_attention(q, keys, values, length, D ** -0.5)
    torch.cuda.synchronize()
    order.append(f"prefill_attention_b{batch}_t{length}")
    del q, keys, values
    print(json.dumps({"profile": list(KERNELS), "projections": order, "launches": launches,
                      "calibration_bytes": CALIBRATION_BYTES}), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode configs")
    ap.add_argument("--no-proj", action="store_true",
                    help="skip the decode projections and decode attention")
    ap.add_argument("--no-prefill-attention", action="store_true",
                    help="skip the causal prefill attention beside torch's flash kernel")
    ap.add_argument("--no-engine", action="store_true",
                    help="skip the end-to-end Qwen3-4B decode through starter_amd.engine")
    ap.add_argument("--engine-workload", metavar="B,T,N",
                    help="run only this engine workload (batch, prompt tokens, new tokens)")
    ap.add_argument("--profile", type=int, default=0, metavar="N",
                    help="only run a calibration copy and N eager launches per prefill kernel "
                         "(for rocprofv3 --pmc), then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the fused kernels are per-row and need no "
              "collective; run with --gpus 1 (multi-GPU sharding is a design note only).",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.profile:
        with torch.inference_mode():
            profile_run(device, args.profile)
        return 0
    print(f"bench: device {torch.cuda.get_device_name(device)}", file=sys.stderr, flush=True)

    with torch.inference_mode():
        copy_gbps = copy_bandwidth(device)
        print(f"bench: copy {copy_gbps:.0f} GB/s", file=sys.stderr, flush=True)
        work = Workload(device)
        torch.cuda.synchronize()
        print(f"bench: buffer sets {work.sets}", file=sys.stderr, flush=True)
        durations = kernel_durations(work, calls=GRAPH_CALLS, replays=max(10, args.steps // 10))
        wall, gpu_seconds = run_prefill_step(work, args.steps, args.warmup)
        ms_per_step = wall * 1e3 / args.steps
        step_bytes = sum(BYTES.values())
        kernels = {}
        for name in KERNELS:
            d = durations[name]
            mean_us, median_us = statistics.fmean(d), statistics.median(d)
            kernels[name] = {
                "us_per_call_median": median_us, "us_per_call_mean": mean_us,
                "bytes_per_call": BYTES[name],
                "gbps": BYTES[name] / (mean_us * 1e3),
                "frac": BYTES[name] / (mean_us * 1e3) / PEAK_GBPS,
                f"{ROW_UNIT[name]}_per_s": ROWS[name] / (mean_us * 1e-6),
                "buffer_sets": work.sets[name],
            }
            print(f"bench: {name:13s} {mean_us:8.2f} us  {kernels[name]['gbps']:7.0f} GB/s "
                  f"({100 * kernels[name]['frac']:.1f}% of peak)", file=sys.stderr, flush=True)
        print(f"bench: step {ms_per_step * 1e3:.1f} us wall, {gpu_seconds * 1e6 / args.steps:.1f} us "
              f"GPU", file=sys.stderr, flush=True)
        del work
        torch.cuda.empty_cache()
        decode = {} if args.no_decode else decode_configs(device)
        for name, entry in decode.items():
            print(f"bench: {name:34s} {entry['us_per_call']:6.2f} us/call", file=sys.stderr,
                  flush=True)
        projections = {} if args.no_proj else decode_projections(device)
        attention = {} if args.no_proj else decode_attention_bench(device)
        prefill_attn = {} if args.no_prefill_attention else prefill_attention_bench(device)
    workloads = ENGINE_WORKLOADS
    if args.engine_workload:
        workloads = (tuple(int(v) for v in args.engine_workload.split(",")),)
    engine = {} if args.no_engine else engine_decode(device, workloads=workloads)

    dominant = max(KERNELS, key=lambda n: kernels[n]["us_per_call_mean"])
    roofline = {"kernel": dominant, "bound": "hbm", "achieved": kernels[dominant]["gbps"],
                "peak": PEAK_GBPS, "unit": "GB/s", "frac": kernels[dominant]["frac"],
                "traffic": pmc_traffic(dominant), "algorithmic_bytes": BYTES[dominant]}
    for name in KERNELS:
        kernels[name]["hbm_bytes_pmc"] = pmc_traffic(name)
    result = {
        "metric": METRIC,
        "value": step_bytes / (ms_per_step * 1e6),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "prefill hot path, 4 x 2048 tokens: embedding gather + "
                               "residual-add RMSNorm + packed QK-norm/RoPE/KV-cache write + "
                               "SiLU*up (BASELINE configs 4a, 4b, 5a, 5b)",
                   "tokens": TOKENS, "hidden": H, "intermediate": I, "vocab": V,
                   "heads": [NQ, NK, D], "step_bytes": step_bytes},
        "frac_of_peak": step_bytes / (ms_per_step * 1e6) / PEAK_GBPS,
        "roofline": roofline,
        "kernels": kernels,
        "decode": decode,
        "projections": projections,
        "attention": attention,
        "prefill_attention": prefill_attn,
        "engine": engine,
        "copy_gbps": copy_gbps,
    }
    if not args.no_cpu:
        print("bench: reference PyTorch formulas on the CPU, per config and whole step ...",
              file=sys.stderr, flush=True)
        reference = torch_cpu_configs()
        result["cpu_reference"] = reference
        step = reference["step"]
        result["cpu_baseline"] = {
            "value": step["gbps"], "unit": "GB/s", "cores": reference["threads"], "kind": "port",
            "sample": (f"the reference's PyTorch formulas (Qwen3RMSNorm, residual add, per-head "
                       f"norm + apply_rotary_pos_emb with the K/V cache fill, F.silu(gate) * up, "
                       f"F.embedding) on bf16 CPU tensors, the whole 4 x 2048-token step, "
                       f"{reference['threads']} threads, median of {step['reps']} after one "
                       f"warm-up: {step['seconds'] * 1e3:.1f} ms/step"),
            "cpu": reference["cpu"], "host_cpus": reference["host_cpus"]}
        print("bench: CPU baseline (C oracle, one thread) ...", file=sys.stderr, flush=True)
        result["cpu_baseline_oracle"] = cpu_baseline()
        gpu_us = {"config1_rms_norm_8x2560": decode.get("config1_rms_norm_8x2560", {}).get("us_per_call"),
                  "config2_add_rms_norm_64x2560_x36":
                      decode.get("config2_add_rms_norm_64x2560_x36", {}).get("us_per_call"),
                  "config3_qk_norm_rope_b32": decode.get("config3_qk_norm_rope_b32", {}).get("us_per_call"),
                  "config4a_add_rms_norm_8192x2560": kernels["add_rms_norm"]["us_per_call_mean"],
                  "config4b_prefill_qkv_4x2048": kernels["prefill_qkv"]["us_per_call_mean"],
                  "config5a_silu_mul_8192x9728": kernels["silu_mul"]["us_per_call_mean"],
                  "config5b_embedding_8192_ids": kernels["embedding"]["us_per_call_mean"]}
        for name, entry in result["cpu_reference"]["configs"].items():
            if gpu_us.get(name):
                entry["gpu_us_per_call"] = gpu_us[name]
            print(f"bench: cpu {name:34s} {entry['us_per_call']:12.1f} us/call "
                  f"({result['cpu_reference']['threads']} threads)", file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
