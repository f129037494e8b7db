"""The fused Q/K/V prologue + decode attention (SmallQueryAttention.run_qkv)
on the MI355X.

Contract: one fused call equals the pair the reference's decode step issues
(engine/decode_step.py:43-47) - qkv_norm_rope_cache, then the attention on
its Q - bit for bit: the same output and the same caches, with the new K/V
row at slot `position` and every other slot untouched (NaN-poisoned tails
stay NaN, and stay unread).  Covered: bf16 rows and f32 split-K partials,
group widths 1..16 (16 takes two launches), the new key at the start, middle,
end and segment boundaries of the attended range and outside it, invalid
positions, and HIP-graph replays with the position advanced on the device.
The composition itself is checked against the float64 oracle pair.
"""

from __future__ import annotations

import pytest
import torch

from conftest import O, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels.decode_fused import qkv_norm_rope_cache  # noqa: E402
from starter_amd.kernels.rotary import default_inv_freq, rope_tables  # noqa: E402
from starter_amd.kernels.small_query_attention import SmallQueryAttention  # noqa: E402

DEV = "cuda"
SCALE = 128 ** -0.5
INV_FREQ = default_inv_freq(5_000_000.0, 128)


def inputs(b, hq, hk, cap, splits, seed):
    g = gen(seed)
    width = (hq + 2 * hk) * 128
    if splits:
        qkv = torch.randn((splits, b, width), generator=g) * 0.7
    else:
        qkv = normal((b, width), g=g)
    qw, kw = normal((128,), 1.0, 0.1, g), normal((128,), 1.0, 0.1, g)
    k, v = normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    return qkv, qw, kw, k, v


def poison(t, used):
    b, hk, cap, d = t.shape
    t = t.clone()
    for vh in range(b * hk):
        t.view(b * hk, cap, d)[vh, int(used[vh]):] = float("nan")
    return t


def pair_and_fused(plan, qkv, qw, kw, cos, sin, pos, k, v, used):
    """(unfused out, caches), (fused out, caches) from identical inputs."""
    k1, v1, k2, v2 = k.clone(), v.clone(), k.clone(), v.clone()
    position = torch.tensor([pos], dtype=torch.int64, device=DEV)
    with torch.inference_mode():
        q = qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k1, v1)
        ref = plan.run(q, k1, v1, used, SCALE)
        out = plan.run_qkv(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k2, v2, used, SCALE)
    return (ref, k1, v1), (out, k2, v2)


CASES = (  # b, hq, hk, cap, qkv splits, position, used rule
    (1, 32, 8, 545, 8, 544, "pos+1"),       # Qwen3-4B batch 1: the new key is the last one
    (4, 32, 8, 300, 8, 150, "pos+1"),
    (2, 8, 2, 129, 0, 0, "pos+1"),          # bf16 rows, first slot
    (1, 16, 1, 193, 16, 64, "pos+1"),       # two launches of 8 query rows; segment boundary
    (3, 6, 2, 257, 4, 63, "mixed"),         # some heads attend past pos, some stop before it
    (1, 4, 4, 64, 1, 63, "pos+1"),          # one query row per kv head
    (2, 4, 2, 100, 2, 99, "mixed"),
    (16, 32, 8, 641, 4, 640, "pos+1"),      # Qwen3-4B batch 16
    (1, 32, 8, 545, 0, 544, "pos+1"),       # Qwen3-4B batch 1 from bf16 rows (the folded step)
    (3, 6, 2, 257, 0, 63, "empty"),         # bf16 rows; mixed lengths and a head with no key
    (2, 4, 2, 100, 3, 99, "empty"),         # the same from three split-K partials
)


@pytest.mark.parametrize("b,hq,hk,cap,splits,pos,rule", CASES)
def test_fused_equals_the_call_pair_bit_for_bit(b, hq, hk, cap, splits, pos, rule):
    qkv, qw, kw, k, v = inputs(b, hq, hk, cap, splits, 700 + cap + hq + splits)
    if rule == "pos+1":
        used = torch.full((b * hk,), pos + 1, dtype=torch.int32)
    else:
        used = torch.arange(b * hk, dtype=torch.int32) * 53 % (cap + 1)
        used[0] = pos + 1
        if rule == "empty":
            used[1] = 0  # a head with no key: zeros, and no NaN from the poisoned cache
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    kp, vp = poison(k, used).to(DEV), poison(v, used).to(DEV)
    args = (qkv.to(DEV), qw.to(DEV), kw.to(DEV), cos, sin, pos, kp, vp, used.to(DEV))
    (ref, k1, v1), (out, k2, v2) = pair_and_fused(plan, *args)
    assert bool(torch.isfinite(out.float()).all())
    assert_bits_exact(out, ref, "attention output")
    assert_bits_exact(k2, k1, "key cache")
    assert_bits_exact(v2, v1, "value cache")
    assert not torch.equal(k2.cpu()[:, :, pos], kp.cpu()[:, :, pos])  # the slot was written
    for t, old in ((args[0], qkv), (args[1], qw), (args[2], kw)):
        assert torch.equal(t.cpu(), old)


def test_fused_matches_the_float64_oracle_pair():
    b, hq, hk, cap, splits, pos = 2, 32, 8, 300, 8, 211
    qkv, qw, kw, k, v = inputs(b, hq, hk, cap, splits, 790)
    used = torch.full((b * hk,), pos + 1, dtype=torch.int32)
    used[3] = 17  # a head that stops before the new key
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    kd, vd = k.to(DEV), v.to(DEV)
    with torch.inference_mode():
        out = plan.run_qkv(qkv.to(DEV), qw.to(DEV), kw.to(DEV), 1e-6, 2e-6, cos, sin,
                           torch.tensor([pos], device=DEV), kd, vd, used.to(DEV), SCALE)
    eq, ek, ev = O.qkv_norm_rope_cache(qkv.numpy(), bits(qw), bits(kw), 1e-6, 2e-6, bits(cos),
                                       bits(sin), pos, bits(k), bits(v))
    assert_bits_exact(kd, ek, "key cache")      # the Q/K/V half is bit-exact
    assert_bits_exact(vd, ev, "value cache")
    ref = torch.from_numpy(O.bf16_value(O.decode_attention(eq, ek, ev, used.numpy(), SCALE)))
    torch.testing.assert_close(out.float().cpu(), ref, rtol=0.02, atol=0.004)


@pytest.mark.parametrize("pos", [-1, 97])
def test_invalid_position_writes_nothing(pos):
    """Out-of-range positions leave both caches untouched (the queries are
    NaN, as qkv_norm_rope_cache returns them); the fused call still equals
    the pair."""
    b, hq, hk, cap = 2, 8, 2, 97
    qkv, qw, kw, k, v = inputs(b, hq, hk, cap, 4, 800)
    used = torch.full((b * hk,), 50, dtype=torch.int32)
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    args = (qkv.to(DEV), qw.to(DEV), kw.to(DEV), cos, sin, pos, k.to(DEV), v.to(DEV), used.to(DEV))
    (ref, k1, v1), (out, k2, v2) = pair_and_fused(plan, *args)
    assert_bits_exact(out, ref, "output")
    assert torch.equal(k2.cpu(), k) and torch.equal(v2.cpu(), v)


def test_graph_replays_follow_the_device_position():
    """Captured once, replayed with position / used advanced on the device, as
    the engine's decode graph does; each replay matches the eager pair."""
    b, hq, hk, cap = 2, 32, 8, 160
    qkv, qw, kw, k, v = inputs(b, hq, hk, cap, 8, 810)
    qkv, qw, kw = qkv.to(DEV), qw.to(DEV), kw.to(DEV)
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    k1, v1, k2, v2 = (t.to(DEV) for t in (k, v, k, v))
    position = torch.tensor([5], dtype=torch.int64, device=DEV)
    used = torch.full((b * hk,), 6, dtype=torch.int32, device=DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    run = lambda: plan.run_qkv(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k2, v2, used, SCALE)  # noqa: E731
    with torch.inference_mode(), torch.cuda.stream(stream):
        run()                                   # warm-up: writes slot 5 of k2 / v2 ...
    torch.cuda.current_stream().wait_stream(stream)
    with torch.inference_mode():                # ... and the pair writes it in k1 / v1
        plan.run(qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k1, v1),
                 k1, v1, used, SCALE)
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph, stream=stream):
        out = run()
    with torch.inference_mode():
        for pos in (6, 7, 63, 64, 65, 159):
            position.fill_(pos)
            used.fill_(pos + 1)
            graph.replay()
            q = qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k1, v1)
            ref = plan.run(q, k1, v1, used, SCALE)
            torch.cuda.synchronize()
            assert_bits_exact(out, ref, f"replay at {pos}")
            assert_bits_exact(k2, k1, f"key cache at {pos}")
            assert_bits_exact(v2, v1, f"value cache at {pos}")
