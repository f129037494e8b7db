"""The normalising matrix-core projections (``skinny_gemm.linear_partials_normed``
and ``linear_silu_mul_normed``) on the MI355X.

Parity bar: bit-exact.  Each workgroup normalises its slice of the residual
stream from the per-workgroup sums of squares the residual producer
(``row_gemv.linear_residual``) wrote, with ``add_rms_norm``'s rounding steps,
and then runs the tiles, waves and chunk order of the plain entry point; so
the output must equal the plain call on the normalised row bit for bit, and
that row must equal the CPU oracle's RMSNorm of the same total (the plain
calls themselves are pinned against the oracle in test_gpu_skinny.py).
"""

from __future__ import annotations

import pytest
import torch

from conftest import O, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels import row_gemv as rg  # noqa: E402
from starter_amd.kernels import skinny_gemm as sk  # noqa: E402
from starter_amd.kernels.rmsnorm import rms_norm  # noqa: E402

DEV = "cuda"


def residual_stream(rows, width, seed):
    """(total, sq, gain) as the decode step hands them over: total and its
    per-workgroup sums of squares from the real producer (a projection with
    the residual add; width = 256 c for a column count c it serves), and an
    RMSNorm gain."""
    g = gen(seed)
    k_in = 512
    x = normal((rows, k_in), g=g).to(DEV)
    w = normal((width, k_in), std=0.05, g=g).to(DEV)
    residual = normal((rows, width), std=2.0, g=g).to(DEV)
    gain = normal((width,), mean=1.0, std=0.1, g=g).to(DEV)
    total, sq = rg.linear_residual(x, w, residual)
    return total, sq, gain


def normed_row(total, gain, eps):
    """The row add_rms_norm would write, checked against the oracle."""
    normed = rms_norm(total, gain, eps)
    torch.cuda.synchronize()
    assert_bits_exact(normed, O.rms_norm(bits(total.cpu()), bits(gain.cpu()), eps), "normed row")
    return normed


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", [(6144, 2560), (2560, 4096), (512, 512), (2048, 6144)])
def test_partials_normed_is_norm_then_partials(rows, n, k):
    eps = 1e-6
    total, sq, gain = residual_stream(rows, k, 1300 + rows + n)
    w = normal((n, k), std=0.05, g=gen(1400 + n + k)).to(DEV)
    got = sk.linear_partials_normed(total, sq, gain, eps, w)
    want = sk.linear_partials(normed_row(total, gain, eps), w)
    torch.cuda.synchronize()
    assert got.shape == want.shape == (sk.split_count(n, k, rows), rows, n)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), f"rows={rows} n={n} k={k}"


@pytest.mark.parametrize("rows", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", [(9728, 2560), (512, 512), (1024, 1024)])
def test_silu_mul_normed_is_norm_then_silu_mul(rows, n, k):
    eps = 1e-6
    total, sq, gain = residual_stream(rows, k, 1500 + rows + n)
    gate_up = normal((2 * n, k), std=0.05, g=gen(1600 + n + k)).to(DEV)
    got = sk.linear_silu_mul_normed(total, sq, gain, eps, gate_up)
    want = sk.linear_silu_mul(normed_row(total, gain, eps), gate_up)
    torch.cuda.synchronize()
    assert got.shape == want.shape == (rows, n)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"rows={rows} n={n} k={k}"


def test_zero_row_and_large_eps():
    """A zero residual row normalises to zeros (inv = 1/sqrt(eps)); a large
    eps changes every normalised value - both still match the two-call path."""
    rows, n, k = 2, 512, 2560
    total, sq, gain = residual_stream(rows, k, 1700)
    total[1].zero_()
    sq[1].zero_()
    w = normal((n, k), std=0.05, g=gen(1701)).to(DEV)
    gate_up = normal((2 * n, k), std=0.05, g=gen(1702)).to(DEV)
    for eps in (1e-6, 0.5):
        normed = normed_row(total, gain, eps)
        got = sk.linear_partials_normed(total, sq, gain, eps, w)
        assert torch.equal(got.view(torch.int32), sk.linear_partials(normed, w).view(torch.int32))
        got = sk.linear_silu_mul_normed(total, sq, gain, eps, gate_up)
        assert torch.equal(got.view(torch.int16), sk.linear_silu_mul(normed, gate_up).view(torch.int16))


def test_inputs_unchanged_and_shape_rule():
    rows, n, k = 1, 6144, 2560
    total, sq, gain = residual_stream(rows, k, 1800)
    w = normal((n, k), std=0.05, g=gen(1801)).to(DEV)
    before = (total.clone(), sq.clone(), gain.clone())
    sk.linear_partials_normed(total, sq, gain, 1e-6, w)
    torch.cuda.synchronize()
    for a, b in zip(before, (total, sq, gain)):
        assert torch.equal(a, b)
    assert sk.supports_normed_shape(4, 2560, 6144) and sk.supports_normed_shape(4, 2560, 9728, True)
    assert not sk.supports_normed_shape(5, 2560, 6144)
    assert not sk.supports_normed_shape(4, 2570, 6144) and not sk.supports_normed_shape(4, 2560, 6160)
    assert not sk.supports_normed_shape(4, 4096, 2560, True)  # 16,384 slice values per workgroup
    with pytest.raises(ValueError):
        sk.linear_partials_normed(total, sq[:, :128].contiguous(), gain, 1e-6, w)
    with pytest.raises(ValueError):
        sk.linear_partials_normed(total, sq, gain, float("nan"), w)
    with pytest.raises(ValueError):
        sk.linear_silu_mul_normed(total.repeat(5, 1), sq.repeat(5, 1), gain, 1e-6,
                                  normal((1024, k), g=gen(1802)).to(DEV))


@torch.inference_mode()
def test_graph_replay_follows_fresh_inputs():
    """The residual producer and both normalising tiles captured in one HIP
    graph (as in the batch-2 decode step): every replay with new inputs, with
    eager work between the replays, equals the eager calls bit for bit."""
    rows, k_in, width = 2, 512, 2560
    g = gen(1900)
    x = normal((rows, k_in), g=g).to(DEV)
    w_res = normal((width, k_in), std=0.05, g=g).to(DEV)
    residual = normal((rows, width), std=2.0, g=g).to(DEV)
    gain = normal((width,), mean=1.0, std=0.1, g=g).to(DEV)
    w_qkv = normal((1024, width), std=0.05, g=g).to(DEV)
    gate_up = normal((2 * 1024, width), std=0.05, g=g).to(DEV)

    def step():
        total, sq = rg.linear_residual(x, w_res, residual)
        return (sk.linear_partials_normed(total, sq, gain, 1e-6, w_qkv),
                sk.linear_silu_mul_normed(total, sq, gain, 1e-6, gate_up))

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outputs = step()
    torch.cuda.synchronize()
    for replay in range(4):
        x.copy_(normal((rows, k_in), g=g).to(DEV))
        residual.copy_(normal((rows, width), std=2.0, g=g).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        want = step()
        torch.cuda.synchronize()
        assert torch.equal(outputs[0].view(torch.int32), want[0].view(torch.int32)), replay
        assert torch.equal(outputs[1].view(torch.int16), want[1].view(torch.int16)), replay
