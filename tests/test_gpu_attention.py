"""Decode attention on the MI355X against the float64 oracle.

Parity bar: the reference's own acceptance for its kernel against float64
attention (rtol 0.02, atol 0.004; tests/test_small_query_attention.py:232-253)
- the kernel rounds the probabilities that multiply V to bf16, as the
reference does, so it is not the exactly rounded float64 result - plus exact
equality on the known answers where that rounding is exact (uniform weights,
one dominant block), under every split plan.  Unused
cache slots are NaN-poisoned in every case: they must never be read.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import O, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels import _lib  # noqa: E402
from starter_amd.kernels.small_query_attention import SmallQueryAttention, partition_keys  # noqa: E402

DEV = "cuda"
SCALE = 128 ** -0.5


def poison(t, used):
    b, hk, cap, d = t.shape
    t = t.clone()
    for vh in range(b * hk):
        t.view(b * hk, cap, d)[vh, int(used[vh]):] = float("nan")
    return t


def check(out, q, k, v, used):
    ref = torch.from_numpy(O.bf16_value(O.decode_attention(bits(q), bits(k), bits(v), used.numpy(), SCALE)))
    got = out.float().cpu()
    assert bool(torch.isfinite(got).all())
    torch.testing.assert_close(got, ref, rtol=0.02, atol=0.004)
    return (got - ref).abs().max().item()


CASES = ((1, 4, 1, 1), (1, 4, 1, 63), (1, 4, 1, 65), (1, 32, 8, 544), (2, 6, 2, 257),
         (3, 8, 2, 129), (1, 16, 1, 193), (1, 8, 1, 641), (1, 4, 1, 1025), (4, 32, 8, 2080),
         (16, 32, 8, 640), (1, 1, 1, 65), (1, 8, 1, 300),
         (1, 32, 8, 16400), (2, 32, 8, 8200))  # long contexts: 32 and 16 segments of 512+ keys


@pytest.mark.parametrize("b,hq,hk,cap", CASES)
def test_full_and_partial_lengths_with_poisoned_tails(b, hq, hk, cap):
    g = gen(400 + cap + hq)
    q = normal((b, hq, 1, 128), g=g)
    k, v = normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    for used in (torch.full((b * hk,), cap, dtype=torch.int32),
                 torch.arange(b * hk, dtype=torch.int32) * 37 % (cap + 1)):
        kp, vp = poison(k, used), poison(v, used)
        qd, kd, vd, ud = q.to(DEV), kp.to(DEV), vp.to(DEV), used.to(DEV)
        with torch.inference_mode():
            out = plan.run(qd, kd, vd, ud, SCALE)
        check(out, q, k, v, used)
        for t, old in ((qd, q), (kd, kp), (vd, vp), (ud, used)):
            torch.testing.assert_close(t.cpu(), old, rtol=0, atol=0, equal_nan=True)


def test_known_answers_are_exact():
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 193, 128, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    v[:, :, :64], v[:, :, 64:128], v[:, :, 128:] = 2, 6, 20
    used = torch.tensor([193], dtype=torch.int32)
    plan = SmallQueryAttention(1, 4, 1, 193, DEV)
    with torch.inference_mode():
        out = plan.run(q.to(DEV), k.to(DEV), v.to(DEV), used.to(DEV), SCALE)
    assert_bits_exact(out, O.decode_attention(bits(q), bits(k), bits(v), used.numpy(), SCALE), "uniform")
    q.fill_(32)
    k[:, :, :64], k[:, :, 64:128], k[:, :, 128:] = -32, 0, 32
    with torch.inference_mode():
        out = plan.run(q.to(DEV), k.to(DEV), v.to(DEV), used.to(DEV), SCALE)
    assert bool((out == 20).all())
    with torch.inference_mode():
        out = plan.run(q.to(DEV), k.to(DEV), v.to(DEV), torch.zeros(1, dtype=torch.int32, device=DEV), SCALE)
    assert bool((out == 0).all())


def test_every_split_plan_matches_the_oracle():
    """Any (splits, span) covering the capacity gives the same attention up to
    the bf16 rounding of the probabilities (which depends on each segment's
    running maximum), including empty and one-key heads."""
    g = gen(450)
    b, hq, hk, cap = 2, 32, 8, 1100
    q, k, v = normal((b, hq, 1, 128), g=g), normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    used = torch.tensor([1100, 1, 64, 65, 700, 1099, 0, 513] * 2, dtype=torch.int32)
    qd, kd, vd, ud = q.to(DEV), poison(k, used).to(DEV), poison(v, used).to(DEV), used.to(DEV)
    for splits, align in ((1, 64), (2, 64), (5, 64), (18, 64), (5, 16), (8, 16), (13, 32), (32, 48)):
        span = -(-(-(-cap // align)) // splits) * align   # 16-key multiples are enough
        splits = -(-cap // span)
        part = torch.empty((b * hk, splits, hq // hk, 128), dtype=torch.float32, device=DEV)
        stats = torch.empty((b * hk, splits, 2, hq // hk), dtype=torch.float32, device=DEV)
        out = torch.empty((b, 1, hq, 128), dtype=torch.bfloat16, device=DEV)
        _lib.call("qf_decode_attention", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), ud.data_ptr(),
                  b, hq, hk, cap, SCALE, splits, span, part.data_ptr(), stats.data_ptr(),
                  out.data_ptr(), _lib.stream(qd.device))
        check(out, q, k, v, used)
        assert bool((out.view(b * hk, hq // hk, 128)[6] == 0).all())  # the empty head


@pytest.mark.parametrize("b,cap", [(1, 545), (4, 2081), (16, 641)])
def test_qwen_decode_shapes(b, cap):
    g = gen(460 + b)
    q = normal((b, 32, 1, 128), g=g)
    k, v = normal((b, 8, cap, 128), 0.0, 2.0, g), normal((b, 8, cap, 128), g=g)
    used = torch.randint(1, cap + 1, (b * 8,), generator=g, dtype=torch.int32)
    used[0] = cap
    plan = SmallQueryAttention(b, 32, 8, cap, DEV)
    with torch.inference_mode():
        out = plan.run(q.to(DEV), poison(k, used).to(DEV), poison(v, used).to(DEV), used.to(DEV), SCALE)
    check(out, q, k, v, used)


def test_graph_replay_follows_fresh_lengths():
    """A captured decode step replays attention with the lengths the engine
    writes into `used` before each replay (engine/flash_decode.py:59-72)."""
    g = gen(470)
    b, hq, hk, cap = 2, 32, 8, 300
    q, k, v = normal((b, hq, 1, 128), g=g), normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    used = torch.full((b * hk,), 10, dtype=torch.int32, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode(), torch.cuda.stream(stream):
        for _ in range(2):
            plan.run(qd, kd, vd, used, SCALE)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph, stream=stream):
        out = plan.run(qd, kd, vd, used, SCALE)
    for n in (11, 64, 65, 299, 300, 1):
        used.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        check(out, q, k, v, used.cpu())
        with torch.inference_mode():
            eager = plan.run(qd, kd, vd, used, SCALE)
        assert torch.equal(out, eager)
