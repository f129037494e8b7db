"""Where the decode attention's time goes, phase by phase, on the GPU.

Runs the instrumented build of the fused decode attention
(``qf_decode_attention_qkv_phases`` in ``kernels/libqwen_fused_phases.so``,
the product kernels compiled with ``-DQF_PHASE_STAMPS``) at the engine's
shapes: the Qwen3-4B heads (32 query, 8 key/value, width 128), the whole
cache used, the new token's Q/K/V row coming from the qkv projection as the
engine's decode step hands it over (bf16 rows at batch 1, f32 split-K
partials beyond).  Every attention workgroup stamps the 100 MHz constant
clock (``s_memrealtime``) at eight phase boundaries, every merge workgroup at
three; the calls run back to back in one HIP graph, the K/V caches rotating
over copies larger than the Infinity Cache, as the benchmark times them.

Printed per shape, as medians over calls (and over workgroups where a phase
is per workgroup), in microseconds:

* the call's span (first attention workgroup starts -> last merge workgroup
  done) and the plain kernels' time per call in the same graph shape,
  without stamps;
* the dispatch spread (first to last attention workgroup start);
* per attention workgroup: entry -> ``used``/position loaded -> prologue and
  first key loads issued -> queries ready (barrier) -> first key block
  consumed -> key loop done -> waves merged -> stored and acknowledged;
* the gap from the last attention workgroup's end to the first merge
  workgroup's start (the launch hand-off), and the merge's own phases
  (entry -> its loads landed -> merged -> stored and acknowledged);
* the gap from one call's merge end to the next call's first start.

Run: ``python -m starter_amd.attention_phases`` (needs an MI355X and the
built libraries).
"""

from __future__ import annotations

import argparse
import ctypes
import statistics
import sys

import torch

from .kernels import _lib
from .kernels.rotary import default_inv_freq, rope_tables
from .engine import KEY_ALIGN
from .kernels.small_query_attention import SmallQueryAttention

NQ, NK, D = 32, 8, 128
PHASES = 16
MERGE_PHASES = 4
#: hipDeviceAttributeWallClockRate (hip_runtime_api.h): the s_memrealtime clock in kHz
_WALL_CLOCK_RATE = 10017
#: (batch, cache length, split-K partials of the qkv row; 0 = bf16 rows), as
#: the engine's decode step hands them over: bf16 rows from the folded
#: projection at batch 1, the split-K plan's 8 and 4 partials at 4 and 16
CASES = ((1, 545, 0), (4, 2081, 8), (16, 641, 4))
PHASE_NAMES = ("used/pos loaded", "prologue + keys issued", "queries ready",
               "first block consumed", "key loop done", "waves merged", "stored")
#: wave 0's phases 5 -> 6 split at the barrier before the merge
BARRIER_NAMES = ("last wave's loop done (after wave 0's)", "barrier passed", "wave 0 merged")


def _phases_lib():
    lib = ctypes.CDLL(str(_lib.LIBRARY.with_name("libqwen_fused_phases.so")))
    vp, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
    fn = lib.qf_decode_attention_qkv_phases
    fn.argtypes = [vp, i32, vp, vp, f32, f32, vp, vp, vp, vp, vp, vp, i64, i32, i32, i64, f32, i32,
                   i64, vp, vp, vp, vp, vp]
    fn.restype = i32
    return fn


def _clock_mhz(device: int = 0) -> float:
    """The constant clock s_memrealtime counts, from the HIP runtime torch uses."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    value = ctypes.c_int()
    st = hip.hipDeviceGetAttribute(ctypes.byref(value), _WALL_CLOCK_RATE, device)
    if st != 0 or value.value <= 0:
        raise RuntimeError(f"hipDeviceGetAttribute(WallClockRate) failed ({st})")
    return value.value / 1e3


def _sets(nbytes: int) -> int:
    """Copies of the K/V caches whose total exceeds twice the 256 MB Infinity Cache."""
    return max(2, -(-2 * 256 * 2**20 // nbytes) + 1)


def measure(batch: int, keys: int, qkv_splits: int, calls: int = 24, replays: int = 20,
            device: str = "cuda") -> dict:
    fn = _phases_lib()
    clock = _clock_mhz(torch.device(device).index or 0)
    g = torch.Generator(device=device).manual_seed(batch * 1000 + keys)

    def normal(shape, mean=0.0, std=1.0):
        return (torch.randn(shape, generator=g, device=device) * std + mean).to(torch.bfloat16)

    plan = SmallQueryAttention(batch, NQ, NK, keys, device, key_align=KEY_ALIGN)  # the Engine's plan
    vheads, splits = batch * NK, plan.splits
    width = (NQ + 2 * NK) * D
    kv_bytes = 2 * batch * NK * keys * D * 2
    sets = _sets(kv_bytes)
    caches = [(normal((batch, NK, keys, D)), normal((batch, NK, keys, D))) for _ in range(sets)]
    qkv = (normal((batch, width)) if qkv_splits == 0 else
           torch.randn((qkv_splits, batch, width), generator=g, device=device) / qkv_splits)
    qw, kw = normal((D,), 1.0, 0.1), normal((D,), 1.0, 0.1)
    cos, sin = rope_tables(default_inv_freq(5e6, D).to(device), keys, device=device)
    position = torch.full((1,), keys - 1, dtype=torch.int64, device=device)
    used = torch.full((vheads,), keys, dtype=torch.int32, device=device)
    out = torch.empty((batch, 1, NQ, D), dtype=torch.bfloat16, device=device)
    merge_blocks = -(-vheads * (NQ // NK) // 4) if splits > 1 else 0
    per_call = vheads * splits * PHASES + merge_blocks * MERGE_PHASES
    stamps = torch.zeros((calls, per_call), dtype=torch.int64, device=device)
    scale = D ** -0.5

    def call(i, stamped=True):
        k, v = caches[i % sets]
        args = (qkv.data_ptr(), qkv_splits, qw.data_ptr(), kw.data_ptr(), 1e-6, 1e-6,
                cos.data_ptr(), sin.data_ptr(), position.data_ptr(), k.data_ptr(), v.data_ptr(),
                used.data_ptr(), batch, NQ, NK, keys, scale, splits, plan.span,
                plan.partials.data_ptr(), plan.stats.data_ptr(), out.data_ptr())
        stream = _lib.stream(torch.device(device))
        if stamped:
            st = fn(*args, stamps[i].data_ptr(), stream)
        else:
            st = _lib.lib().qf_decode_attention_qkv(*args, stream)
        if st != 0:
            raise RuntimeError(f"attention call failed: {_lib.lib().qf_error_string(st)}")

    def graph_of(stamped):
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for i in range(calls):
                call(i, stamped)
        torch.cuda.current_stream(device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(calls):
                call(i, stamped)
        return graph

    # the plain kernels' time per call, same graph shape, no stamps
    plain = graph_of(False)
    for _ in range(3):
        plain.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        plain.replay()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / calls)
    plain_us = statistics.median(times)

    stamped = graph_of(True)
    rows = {name: [] for name in ("span", "spread", "handoff", "next_call", "merge_load",
                                  "merge_combine",
                                  "merge_store", "attention_span", "first_block_spread",
                                  *PHASE_NAMES, *BARRIER_NAMES)}
    for _ in range(replays):
        stamps.zero_()
        stamped.replay()
        torch.cuda.synchronize()
        host = stamps.cpu()
        prev_end = None
        for i in range(calls):
            row = host[i]
            att = row[:vheads * splits * PHASES].view(vheads * splits, PHASES).double()
            first = float(att[:, 0].min())
            att_end = float(att[:, 7].max())
            rel = (att - first) / clock
            for p, name in enumerate(PHASE_NAMES, start=1):
                rows[name].extend((rel[:, p] - rel[:, p - 1]).tolist())
            last_loop = rel[:, 8:12].max(1).values
            rows[BARRIER_NAMES[0]].extend((last_loop - rel[:, 5]).tolist())
            rows[BARRIER_NAMES[1]].extend((rel[:, 12] - last_loop).tolist())
            rows[BARRIER_NAMES[2]].extend((rel[:, 6] - rel[:, 12]).tolist())
            firsts = torch.cat([rel[:, 4:5], rel[:, 13:16]], 1)
            rows["first_block_spread"].extend((firsts.max(1).values - firsts.min(1).values).tolist())
            rows["spread"].append(float(rel[:, 0].max()))
            rows["attention_span"].append((att_end - first) / clock)
            end = att_end
            if merge_blocks:
                mer = row[vheads * splits * PHASES:].view(merge_blocks, MERGE_PHASES).double()
                rows["handoff"].append((float(mer[:, 0].min()) - att_end) / clock)
                rows["merge_load"].extend(((mer[:, 3] - mer[:, 0]) / clock).tolist())
                rows["merge_combine"].extend(((mer[:, 1] - mer[:, 3]) / clock).tolist())
                rows["merge_store"].extend(((mer[:, 2] - mer[:, 1]) / clock).tolist())
                end = float(mer[:, 2].max())
            rows["span"].append((end - first) / clock)
            if prev_end is not None:
                rows["next_call"].append((first - prev_end) / clock)
            prev_end = end
    result = {"batch": batch, "keys": keys, "splits": splits, "qkv_splits": qkv_splits,
              "plain_us_per_call": plain_us, "clock_mhz": clock}
    for name, values in rows.items():
        if values:
            result[name] = (statistics.median(values), max(values))
    del caches
    torch.cuda.empty_cache()
    return result


def table(results) -> str:
    head = "| phase (µs; median / max over workgroups and calls) | " + " | ".join(
        f"b{r['batch']} × {r['keys']} ({r['splits']} seg.)" for r in results) + " |"
    lines = [head, "|---" * (len(results) + 1) + "|"]

    def line(label, key, both=True):
        cells = []
        for r in results:
            if key not in r:
                cells.append("—")
            elif both:
                cells.append(f"{r[key][0]:.2f} / {r[key][1]:.2f}")
            else:
                cells.append(f"{r[key][0]:.2f}")
        lines.append(f"| {label} | " + " | ".join(cells) + " |")

    lines.append("| plain kernels per call, same graph (no stamps) | " +
                 " | ".join(f"{r['plain_us_per_call']:.2f}" for r in results) + " |")
    line("call span: first attention start → last merge store (median)", "span", both=False)
    line("attention span: first start → last store", "attention_span")
    line("dispatch spread of the attention workgroups' starts", "spread")
    for p, name in enumerate(PHASE_NAMES, start=1):
        line(f"attention phase {p}: → {name}", name)
    line("  of phase 6: the slowest wave's key loop ends after wave 0's by", BARRIER_NAMES[0])
    line("  of phase 6: barrier passed after the slowest wave's loop", BARRIER_NAMES[1])
    line("  of phase 6: the merge of the four waves", BARRIER_NAMES[2])
    line("spread of the four waves' first-block times", "first_block_spread")
    line("hand-off: last attention store → first merge start", "handoff")
    line("merge: start → its loads landed", "merge_load")
    line("merge: loads landed → merged", "merge_combine")
    line("merge: merged → stored", "merge_store")
    line("next call: last store → next call's first start", "next_call")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--calls", type=int, default=24)
    ap.add_argument("--replays", type=int, default=20)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("attention_phases needs a GPU", file=sys.stderr)
        return 2
    results = []
    for batch, keys, qkv_splits in CASES:
        r = measure(batch, keys, qkv_splits, args.calls, args.replays)
        print(f"phases: b{batch} x {keys}: plain {r['plain_us_per_call']:.2f} us/call, "
              f"stamped span {r['span'][0]:.2f} us", file=sys.stderr, flush=True)
        results.append(r)
    print(f"s_memrealtime clock: {results[0]['clock_mhz']:.1f} MHz; {args.calls} calls per graph, "
          f"{args.replays} replays")
    print(table(results))
    return 0


if __name__ == "__main__":
    sys.exit(main())
