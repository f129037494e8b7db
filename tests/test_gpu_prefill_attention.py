"""Causal prefill attention (``kernels.prefill.prefill_attention``,
``qf_prefill_attention``) on the MI355X against the float64 oracle.

The probabilities are rounded to bf16 before they multiply V (as the flash
kernel the reference calls does), so the result depends on the tile order and
there is no bit-exact target: the bar is the reference's own attention
tolerance against float64 (rtol 0.02, atol 0.004; tests/test_small_query_
attention.py in the reference), and an RMS error below 1% of the RMS output.
Shapes cover 1, 2, 4 and 8 query heads per KV head, prompts that end inside a
query block and inside a key block, one token, and the Qwen3-4B head layout;
cache slots past the prompt hold NaN and must never reach the output.  The
8-wave form's grouped work orders must write every block of an output that
starts as NaN.  Known answers: zero queries give the running mean of V
exactly; inputs stay untouched; a captured graph replays with new contents.  Scores that climb
across key blocks (every block raises the row maxima by more than the lazy
rescale threshold) and that fall (no block after the first raises them), and
negative and zero scales (Q enters negated, exact in bf16), cover the
rescaling branches.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import O, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels.prefill import prefill_attention  # noqa: E402

DEV = "cuda"
SCALE = 128 ** -0.5


def operands(b, t, hq, hk, cap, seed, poison=True):
    g = gen(seed)
    q = normal((b, t, hq, 128), g=g)
    k, v = normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    if poison:
        k[:, :, t:], v[:, :, t:] = float("nan"), float("nan")
    return q, k, v


def check(got, q, k, v, t, what, scale=SCALE):
    want = O.bf16_value(O.prefill_attention(bits(q), bits(k), bits(v), t, scale))
    have = O.bf16_value(bits(got))
    assert not np.isnan(have).any(), f"{what}: NaN in the output"
    np.testing.assert_allclose(have, want, rtol=0.02, atol=0.004, err_msg=what)
    rel = float(np.sqrt(np.mean((have - want) ** 2)) / np.sqrt(np.mean(want ** 2)))
    assert rel < 0.01, f"{what}: relative RMS error {rel:.4g}"


@pytest.mark.parametrize("b,t,hq,hk,cap", [
    (1, 1, 4, 2, 8),        # one token
    (2, 37, 8, 2, 40),      # G = 4, ends inside a query block
    (1, 70, 4, 4, 96),      # G = 1 (two waves of each workgroup idle)
    (3, 33, 8, 4, 50),      # G = 2
    (1, 64, 16, 2, 64),     # G = 8, capacity = length
    (1, 200, 32, 8, 256),   # Qwen3-4B heads, several key blocks
    (2, 129, 32, 8, 130),   # one position past a key block
    (3, 333, 32, 8, 340),   # 4-wave form over 16-position blocks, 6 key blocks
    (1, 700, 32, 8, 704),   # ... 11 key blocks, rescales across many blocks
])
def test_matches_oracle(b, t, hq, hk, cap):
    q, k, v = operands(b, t, hq, hk, cap, 800 + t + hq)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    snapshot = [x.clone() for x in (qd, kd, vd)]
    out = prefill_attention(qd, kd, vd, t, SCALE)
    torch.cuda.synchronize()
    assert out.shape == (b, t, hq, 128) and out.dtype == torch.bfloat16
    check(out, q, k, v, t, f"b{b} t{t} hq{hq} hk{hk}")
    for before, after in zip(snapshot, (qd, kd, vd)):   # inputs untouched
        assert torch.equal(before.view(torch.int16), after.view(torch.int16))


@pytest.mark.parametrize("scale", [-SCALE, 0.0, 3 * SCALE])
def test_other_scales(scale):
    b, t, hq, hk, cap = 2, 150, 8, 2, 160
    q, k, v = operands(b, t, hq, hk, cap, 860)
    out = prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), t, scale)
    check(out, q, k, v, t, f"scale {scale}", scale)


@pytest.mark.parametrize("climb", [True, False])
def test_monotone_scores(climb):
    """Key j = c_j (1, .., 1), q = 1/4: the score of key j is 2 c_j, exact.
    Climbing c_j = j / 16 lifts every row maximum by ~16 (log2 units) per
    block, past the rescale threshold; falling c_j puts the maximum at key 0."""
    b, t, hq, hk = 1, 250, 8, 2
    j = torch.arange(t, dtype=torch.float32)
    c = j / 16 if climb else (t - 1 - j) / 16
    k = c.view(1, 1, t, 1).expand(b, hk, t, 128).to(torch.bfloat16).contiguous()
    q = torch.full((b, t, hq, 128), 0.25).to(torch.bfloat16)
    v = normal((b, hk, t, 128), g=gen(861))
    out = prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), t, SCALE)
    check(out, q, k, v, t, f"climb={climb}")


@pytest.mark.parametrize("b,t,hq,hk,seq,kvh", [
    (4, 2048, 16, 4, 3, 1),   # G = 4: 512 workgroups of 64 positions (8 waves)
    (4, 1024, 32, 4, 1, 3),   # G = 8: 512 workgroups of 32 positions (8 waves)
    (1, 2048, 32, 8, 0, 5),   # G = 4: 256 workgroups, one per CU (8 waves)
])
def test_wide_workgroups_match_oracle_slices(b, t, hq, hk, seq, kvh):
    """Grids of >= 256 workgroups take the 8-wave form; one (sequence, KV
    head) slice of its output against the float64 oracle of that slice."""
    q, k, v = operands(b, t, hq, hk, t + 8, 880 + t + hq)
    out = prefill_attention(q.to(DEV), k.to(DEV), v.to(DEV), t, SCALE)
    torch.cuda.synchronize()
    g = hq // hk
    heads = slice(kvh * g, (kvh + 1) * g)
    check(out[seq:seq + 1, :, heads].cpu(), q[seq:seq + 1, :, heads].contiguous(),
          k[seq:seq + 1, kvh:kvh + 1].contiguous(), v[seq:seq + 1, kvh:kvh + 1].contiguous(), t,
          f"b{b} t{t} hq{hq} hk{hk} slice ({seq}, {kvh})")


@pytest.mark.parametrize("b,t,hq,hk", [
    (16, 512, 32, 8),   # 4 (sequence, KV head) pairs per XCD and group, 4 groups
    (8, 256, 32, 8),    # 4 per group, 2 groups
    (64, 128, 32, 8),   # 8 per group (two query blocks each), 8 groups
    (6, 1024, 32, 8),   # 6 pairs per XCD: groups of 3
    (4, 2048, 32, 8),   # 4 pairs per XCD: the plain order
    (5, 1664, 8, 2),    # 10 pairs, not a multiple of the XCD count: the plain order
])
def test_grouped_work_orders_write_every_block(b, t, hq, hk):
    """The 8-wave form walks the pairs of each XCD a group at a time; every
    (query block, pair) must be computed exactly once.  The whole output,
    written into NaN, against torch's flash kernel."""
    from starter_amd.kernels import _lib
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator(device=DEV).manual_seed(b + t)
    cap = t + 16
    q = torch.randn(b, t, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, hk, cap, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(b, hk, cap, 128, generator=g, device=DEV).to(torch.bfloat16)
    out = torch.full_like(q, float("nan"))
    _lib.call("qf_prefill_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), b, t, hq, hk, cap,
              SCALE, out.data_ptr(), _lib.stream(q.device))
    with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
        ref = torch.nn.functional.scaled_dot_product_attention(
            q.transpose(1, 2), k[:, :, :t], v[:, :, :t], is_causal=True, scale=SCALE,
            enable_gqa=True).transpose(1, 2)
    assert not torch.isnan(out).any()
    torch.testing.assert_close(out.float(), ref.float(), rtol=0.02, atol=0.004)


def test_zero_queries_give_the_running_mean():
    t, hk, hq = 100, 2, 8
    q = torch.zeros(1, t, hq, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(1, hk, t, 128, dtype=torch.bfloat16, device=DEV)
    # V row j = 2j: the mean of rows 0..t is t, exact in bf16 up to 256
    v = (2 * torch.arange(t, dtype=torch.float32, device=DEV)).view(1, 1, t, 1)
    v = v.expand(1, hk, t, 128).to(torch.bfloat16).contiguous()
    out = prefill_attention(q, k, v, t, SCALE).float()
    want = torch.arange(t, dtype=torch.float32, device=DEV).view(1, t, 1, 1).expand_as(out)
    assert torch.equal(out, want)


def test_qwen_prefill_shape_against_torch_flash():
    """4 x 512 tokens with the Qwen3-4B heads, against torch's flash kernel on
    the same tensors (both round P to bf16; they agree to the same tolerance)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator(device=DEV).manual_seed(5)
    b, t, hq, hk = 4, 512, 32, 8
    q = torch.randn(b, t, hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(b, hk, t + 16, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(b, hk, t + 16, 128, generator=g, device=DEV).to(torch.bfloat16)
    out = prefill_attention(q, k, v, t, SCALE)
    with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
        ref = torch.nn.functional.scaled_dot_product_attention(
            q.transpose(1, 2), k[:, :, :t], v[:, :, :t], is_causal=True, scale=SCALE,
            enable_gqa=True).transpose(1, 2)
    torch.testing.assert_close(out.float(), ref.float(), rtol=0.02, atol=0.004)


def test_graph_replay_follows_new_contents():
    b, t, hq, hk, cap = 2, 45, 8, 2, 64
    q, k, v = (x.to(DEV) for x in operands(b, t, hq, hk, cap, 870, poison=False))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        prefill_attention(q, k, v, t, SCALE)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = prefill_attention(q, k, v, t, SCALE)
    for seed in (871, 872, 873):
        nq, nk, nv = operands(b, t, hq, hk, cap, seed, poison=False)
        q.copy_(nq); k.copy_(nk); v.copy_(nv)
        graph.replay()
        torch.cuda.synchronize()
        check(out, nq, nk, nv, t, f"replay seed {seed}")
