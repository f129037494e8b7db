"""o_proj over the unmerged attention segments (skinny_gemm.linear_partials_merged)
on the MI355X.

Contract: ``run_qkv_unmerged`` + ``linear_partials_merged`` equals the pair
the reference's decode step hands over (engine/decode_step.py:48-52) -
the merged attention output, then ``linear_partials`` for o_proj - bit for
bit, with the same caches.  Covered: one and two batches of segments
(S = 2..32), batch 1..16 (16 is the most rows), group widths 1, 4 and 16,
heads with no valid key (zero rows), and a HIP graph replayed with the
position advanced on the device.

Against the oracle directly: the oracle's Q/K/V fold, norm, RoPE and cache
write, its float64 attention rounded to bf16, then its exactly rounded
partials of that attended row.  The attention has no bit-exact target (the
bf16 probabilities make it tile-order dependent), so each partial must lie
within sum_k |W[n, k]| * |a_hip[k] - a_oracle[k]| (what the attention
differences can move it) plus the f32 accumulation bound 2^-16 *
sum_k |W[n, k] * a[k]| of the oracle's, with a_hip within the reference's
attention tolerance of a_oracle; the caches must equal the oracle's bit for
bit.
"""

from __future__ import annotations

import pytest
import torch

import numpy as np

from conftest import O, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels.rotary import default_inv_freq, rope_tables  # noqa: E402
from starter_amd.kernels.skinny_gemm import (  # noqa: E402
    linear_partials, linear_partials_merged, supports_merged)
from starter_amd.kernels.small_query_attention import SmallQueryAttention  # noqa: E402

DEV = "cuda"
SCALE = 128 ** -0.5
INV_FREQ = default_inv_freq(5_000_000.0, 128)


def assert_f32_bits(actual, expected, what):
    assert actual.shape == expected.shape, (what, actual.shape, expected.shape)
    same = actual.view(torch.int32) == expected.view(torch.int32)
    assert bool(same.all()), f"{what}: {int((~same).sum())} of {same.numel()} values differ"


def operands(b, hq, hk, cap, n, seed):
    g = gen(seed)
    qkv = torch.randn((4, b, (hq + 2 * hk) * 128), generator=g) * 0.7
    qw, kw = normal((128,), 1.0, 0.1, g), normal((128,), 1.0, 0.1, g)
    k, v = normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    w = normal((n, hq * 128), 0.0, 0.02, g)
    return [t.to(DEV) for t in (qkv, qw, kw, k, v, w)]


def both_ways(plan, qkv, qw, kw, cos, sin, pos, k, v, used, w):
    """(reference partials, caches), (merged partials, caches)."""
    b = plan.batch
    k1, v1, k2, v2 = k.clone(), v.clone(), k.clone(), v.clone()
    position = torch.tensor([pos], dtype=torch.int64, device=DEV)
    with torch.inference_mode():
        attended = plan.run_qkv(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k1, v1, used, SCALE)
        ref = linear_partials(attended.view(b, -1), w)
        plan.partials.fill_(float("nan"))  # only what the second call writes may be read
        plan.stats.fill_(float("nan"))
        plan.run_qkv_unmerged(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k2, v2, used, SCALE)
        out = linear_partials_merged(plan.partials, plan.stats, b, w)
    return (ref, k1, v1), (out, k2, v2)


CASES = (  # b, hq, hk, cap, n, used rule
    (1, 32, 8, 545, 2560, "full"),     # Qwen3-4B batch 1: 9 segments
    (1, 32, 8, 1100, 2560, "full"),    # 18 segments: two batches in the merge
    (1, 32, 8, 4000, 2560, "full"),    # 32 segments
    (2, 32, 8, 700, 2560, "mixed"),
    (4, 8, 2, 300, 512, "mixed"),      # some heads attend nothing
    (16, 32, 8, 200, 2560, "full"),    # the most rows
    (3, 16, 1, 193, 1024, "full"),     # 16 query rows per kv head
    (2, 4, 4, 150, 256, "mixed"),      # one query row per kv head
)


@pytest.mark.parametrize("b,hq,hk,cap,n,rule", CASES)
def test_merged_projection_equals_merge_then_project(b, hq, hk, cap, n, rule):
    qkv, qw, kw, k, v, w = operands(b, hq, hk, cap, n, 900 + cap + b)
    pos = cap - 1
    if rule == "full":
        used = torch.full((b * hk,), cap, dtype=torch.int32)
    else:
        used = torch.arange(b * hk, dtype=torch.int32) * 97 % (cap + 1)
        used[-1] = 0                      # no valid key: a zero row
        used[0] = cap
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    assert plan.splits > 1 and supports_merged(plan.partials, plan.stats, b, w), plan.splits
    (ref, k1, v1), (out, k2, v2) = both_ways(plan, qkv, qw, kw, cos, sin, pos, k, v,
                                             used.to(DEV), w)
    assert bool(torch.isfinite(out).all())
    assert_f32_bits(out, ref, f"o_proj partials (S={plan.splits})")
    assert_bits_exact(k2, k1, "key cache")
    assert_bits_exact(v2, v1, "value cache")


def test_graph_replays_follow_the_device_position():
    """Captured once and replayed with position / used advanced on the
    device, as the engine's decode graph does; each replay's partials equal
    the eager merge-then-project pair."""
    b, hq, hk, cap, n = 1, 32, 8, 400, 2560
    qkv, qw, kw, k, v, w = operands(b, hq, hk, cap, n, 950)
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    graph_plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    eager_plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    kg, vg, ke, ve = k.clone(), v.clone(), k.clone(), v.clone()
    position = torch.tensor([200], dtype=torch.int64, device=DEV)
    used = torch.full((b * hk,), 201, dtype=torch.int32, device=DEV)

    def step():
        graph_plan.run_qkv_unmerged(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, kg, vg, used, SCALE)
        return linear_partials_merged(graph_plan.partials, graph_plan.stats, b, w)

    with torch.inference_mode():
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            step()  # warm-up writes slot 200 into the graph's caches, as replay 0 does
        torch.cuda.current_stream().wait_stream(stream)
        ke[:, :, 200], ve[:, :, 200] = kg[:, :, 200], vg[:, :, 200]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = step()
        for replay in range(4):
            graph.replay()
            torch.cuda.synchronize()
            p = int(position.item())
            attended = eager_plan.run_qkv(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, ke, ve,
                                          used, SCALE)
            ref = linear_partials(attended.view(b, -1), w)
            torch.cuda.synchronize()
            assert_f32_bits(out, ref, f"replay {replay} (position {p})")
            assert_bits_exact(kg, ke, f"key cache after replay {replay}")
            position.add_(1)
            used.add_(1)


@pytest.mark.parametrize("b,hq,hk,cap,n,rule", [CASES[0], CASES[3], CASES[4], CASES[6]])
def test_merged_projection_against_the_oracle(b, hq, hk, cap, n, rule):
    qkv, qw, kw, k, v, w = operands(b, hq, hk, cap, n, 1900 + cap + b)
    pos = cap - 1
    if rule == "full":
        used = torch.full((b * hk,), cap, dtype=torch.int32)
    else:
        used = torch.arange(b * hk, dtype=torch.int32) * 97 % (cap + 1)
        used[-1] = 0
        used[0] = cap
    cos, sin = rope_tables(INV_FREQ, cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    kh, vh = k.clone(), v.clone()
    position = torch.tensor([pos], dtype=torch.int64, device=DEV)
    with torch.inference_mode():
        plan.run_qkv_unmerged(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, kh, vh,
                              used.to(DEV), SCALE)
        out = linear_partials_merged(plan.partials, plan.stats, b, w)
        # the attended row the merge produced, for the bound below
        attended = plan.run_qkv(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k.clone(),
                                v.clone(), used.to(DEV), SCALE)
    torch.cuda.synchronize()
    q_or, k_or, v_or = O.qkv_norm_rope_cache(qkv.cpu().numpy(), bits(qw), bits(kw), 1e-6, 2e-6,
                                             bits(cos), bits(sin), pos, bits(k), bits(v))
    assert_bits_exact(kh, k_or, "key cache vs oracle")
    assert_bits_exact(vh, v_or, "value cache vs oracle")
    att_or = O.decode_attention(q_or, k_or, v_or, used.numpy(), SCALE)      # bf16 [B, 1, Hq, 128]
    a_or = O.bf16_value(att_or.reshape(b, -1)).astype(np.float64)
    a_hip = O.bf16_value(bits(attended).reshape(b, -1)).astype(np.float64)
    np.testing.assert_allclose(a_hip, a_or, rtol=0.02, atol=0.004)
    splits = out.shape[0]
    want = O.linear_partials(att_or.reshape(b, -1), bits(w), splits).astype(np.float64)
    got = out.cpu().numpy().astype(np.float64)
    wv = np.abs(O.bf16_value(bits(w)).astype(np.float64))                # [N, K]
    span = (hq * 128) // splits
    for s_ in range(splits):
        cols = slice(s_ * span, (s_ + 1) * span)
        moved = np.abs(a_hip[:, cols] - a_or[:, cols]) @ wv[:, cols].T     # [B, N]
        accum = 2.0 ** -16 * (np.abs(a_or[:, cols]) @ wv[:, cols].T)
        err = np.abs(got[s_] - want[s_])
        assert bool((err <= moved + accum + 1e-30).all()), (
            f"split {s_}: worst excess {float((err - moved - accum).max()):.3g}")
