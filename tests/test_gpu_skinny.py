"""Split-K decode projections on the MI355X against the CPU oracle.

Parity bar (the kernels accumulate in f32 on the matrix cores, so only inputs
whose partial sums are exact f32 values have one right answer):

* integer-valued bf16 inputs: every partial sum is an exact f32, so the
  partials and the SiLU * up output must equal the oracle bit for bit - this
  pins the tile, fragment, split and epilogue indexing at every dispatch path
  (M = 1 .. 64, both x layouts) and at the Qwen3-4B shapes;
* random inputs: each partial within 2^-16 * sum|x*w| of the exactly rounded
  oracle partial (f32 accumulation error; a dropped k step or a mismatched
  fragment is ~1/K of the magnitude, far above it); SiLU * up within atol /
  rtol 1e-2 of the oracle with >= 99.9% bit-exact, every other element equal
  to SiLU * up of a gate and an up within 2 bf16 ulps of the exactly rounded
  projections, and within the reference's own tolerances of F.linear
  (tests/test_skinny_gemm.py:403-436).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from conftest import O, assert_bf16_close, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels import _lib, skinny_gemm as sk  # noqa: E402
from starter_amd.kernels.decode_fused import add_rms_norm, qkv_norm_rope_cache, silu_mul  # noqa: E402

DEV = "cuda"
QWEN = {"qkv": (6144, 2560), "o": (2560, 4096), "down": (2560, 9728)}
GATE_UP = (9728, 2560)   # n, k of the packed [2n, k] weight
TOL = 2.0**-16           # per-element bound on |partial - exact| / sum|x*w|


def ints(shape, lo, hi, g):
    return torch.randint(lo, hi + 1, shape, generator=g).to(torch.bfloat16)


def bf16_step(b, steps):
    """bf16 bit patterns ``steps`` representable values above ``b`` (below for
    negative steps), through zero: ordered key = bits for +, -(bits & 0x7fff) for -."""
    b = b.astype(np.int64)
    key = np.where(b < 0x8000, b, -(b & 0x7FFF)) + steps
    return np.where(key >= 0, key, 0x8000 | -key).astype(np.uint16)


def exact_int_partials(x, w, splits):
    """float64 matmul of integer-valued operands: exact, so exactly the oracle."""
    per = x.shape[1] // splits
    xd, wd = x.double(), w.double()
    return torch.stack([xd[:, s * per:(s + 1) * per] @ wd[:, s * per:(s + 1) * per].T
                        for s in range(splits)]).float()


def check_partials(got, x, w):
    splits = got.shape[0]
    ref = O.linear_partials(bits(x), bits(w), splits)
    per = x.shape[1] // splits
    xa, wa = x.double().abs(), w.double().abs()
    scale = torch.stack([xa[:, s * per:(s + 1) * per] @ wa[:, s * per:(s + 1) * per].T
                         for s in range(splits)]).numpy()
    err = np.abs(got.cpu().double().numpy() - ref)
    assert (err <= TOL * scale + 1e-30).all(), float((err / (scale + 1e-30)).max())


@pytest.mark.parametrize("m", [1, 3, 4, 5, 16, 17, 31, 32, 33, 48, 49, 64])
def test_partials_integer_exact_every_path(m):
    g = gen(60 + m)
    n, k = 96, 1024
    x, w = ints((m, k), -4, 4, g), ints((n, k), -3, 3, g)
    xd, wd = x.to(DEV), w.to(DEV)
    for splits in (1, 2, 4, 16, sk.split_count(n, k, m)):  # 16: one chunk per split
        p = torch.empty((splits, m, n), dtype=torch.float32, device=DEV)
        _lib.call("qf_linear_partials", xd.data_ptr(), m, k, wd.data_ptr(), n, splits,
                  p.data_ptr(), _lib.stream(xd.device))
        np.testing.assert_array_equal(p.cpu().numpy(), O.linear_partials(bits(x), bits(w), splits))


@pytest.mark.parametrize("m", [1, 4, 5, 8, 9, 12, 13, 16, 17, 33, 64])  # 12 | 13: half tile | tile pairs
@pytest.mark.parametrize("n", [64, 96])  # 96: the last workgroup has waves past N
def test_silu_mul_integer_exact_every_path(m, n):
    g = gen(80 + m + n)
    k = 640
    x, gu = ints((m, k), -2, 2, g), ints((2 * n, k), -1, 1, g)
    got = sk.linear_silu_mul(x.to(DEV), gu.to(DEV))
    assert_bits_exact(got, O.linear_silu_mul(bits(x), bits(gu)), what=f"silu m={m} n={n}")


@pytest.mark.parametrize("name", sorted(QWEN))
@pytest.mark.parametrize("m", [1, 16, 32, 48, 64])
def test_partials_qwen_shapes_integer_exact(name, m):
    n, k = QWEN[name]
    g = gen(100 + m)
    x, w = ints((m, k), -3, 3, g), ints((n, k), -2, 2, g)
    got = sk.linear_partials(x.to(DEV), w.to(DEV))
    assert got.shape == (sk.split_count(n, k, m), m, n)
    torch.testing.assert_close(got.cpu(), exact_int_partials(x, w, got.shape[0]), rtol=0, atol=0)


@pytest.mark.parametrize("m", [1, 4, 8, 12, 13, 16, 32, 48, 64])
def test_silu_mul_qwen_shape_integer_exact(m):
    n, k = GATE_UP
    g = gen(120 + m)
    x, gu = ints((m, k), -2, 2, g), ints((2 * n, k), -1, 1, g)
    got = sk.linear_silu_mul(x.to(DEV), gu.to(DEV))
    proj = (x.double() @ gu.double().T).float().to(torch.bfloat16)
    assert_bits_exact(got, O.silu_mul(bits(proj)), what=f"gate/up m={m}")


@pytest.mark.parametrize("m", [1, 4, 16, 33, 64])
def test_partials_random_within_f32_accumulation(m):
    g = gen(140 + m)
    for name in ("qkv", "o"):
        n, k = QWEN[name]
        x = normal((m, k), g=g)
        w = normal((n, k), 0.0, 1.0 / k**0.5, g)
        before = (x.clone(), w.clone())
        xd, wd = x.to(DEV), w.to(DEV)
        got = sk.linear_partials(xd, wd)
        check_partials(got, x, w)
        # the reference's own acceptance (tests/test_skinny_gemm.py:403-422)
        expected = F.linear(xd.float(), wd.float())
        torch.testing.assert_close(got.sum(0), expected, rtol=2e-3, atol=2e-3)
        torch.testing.assert_close(got.sum(0).to(torch.bfloat16), F.linear(xd, wd), rtol=1.6e-2, atol=1e-2)
        for t, old in zip((xd, wd), before):
            torch.testing.assert_close(t.cpu(), old, rtol=0, atol=0)
        assert torch.equal(got, sk.linear_partials(xd, wd))  # deterministic


@pytest.mark.parametrize("m,n,k", [(1, 9728, 2560), (4, 9728, 2560), (8, 9728, 2560), (16, 9728, 2560),
                                   (64, 512, 256), (3, 64, 64)])
def test_silu_mul_random_matches_oracle_and_unfused_path(m, n, k):
    g = gen(160 + m)
    x = normal((m, k), g=g)
    w = normal((2 * n, k), 0.0, 4.0 / k**0.5, g)
    xd, wd = x.to(DEV), w.to(DEV)
    got = sk.linear_silu_mul(xd, wd)
    assert got.shape == (m, n) and bool(torch.isfinite(got).all())
    ref = O.linear_silu_mul(bits(x), bits(w))
    # within the stated tolerance everywhere and >= 99.9% bit-exact ...
    assert_bf16_close(got, ref, max_ulp=1 << 16, min_exact=0.999, what="linear_silu_mul")
    # ... and every other element is explained by the projections alone: it
    # equals SiLU * up of a bf16 gate and up each within the f32 accumulation
    # bound 2^-16 * sum|x*w| of the exact projection (plus the bf16 rounding
    # half-ulp).  Near a rounding midpoint that moves a projection by an ulp;
    # where the sum cancels to a small value it can move it by several.
    gb = bits(got)
    diff = np.argwhere(gb != ref)
    if diff.size:
        exact = F.linear(x.double(), w.double()).numpy()
        bound = 2.0 ** -16 * F.linear(x.double().abs(), w.double().abs()).numpy()
        def near(value, slack):
            """bf16 patterns within slack of value, plus the one it rounds to."""
            centre = O.bf16_bits(np.float32([value]))[0]
            cands = [int(bf16_step(np.uint16([centre]), i)[0]) for i in range(-64, 65)]
            vals = O.bf16_value(np.uint16(cands)).astype(np.float64)
            return [c for c, v in zip(cands, vals) if abs(v - value) <= slack + abs(v) * 2.0 ** -8] or [centre]
        unexplained = []
        for row, col in diff:
            gates = near(exact[row, col], bound[row, col])
            ups = near(exact[row, col + n], bound[row, col + n])
            pairs = np.array([[gv, uv] for gv in gates for uv in ups], dtype=np.uint16)
            if not (O.silu_mul(pairs)[:, 0] == gb[row, col]).any():
                unexplained.append((int(row), int(col), float(exact[row, col]),
                                    float(exact[row, col + n]), float(bound[row, col])))
        assert not unexplained, (unexplained[:4], len(diff))
    torch.testing.assert_close(got, silu_mul(F.linear(xd, wd)), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("rows,inner", [(4, 4096), (64, 4096), (64, 9728)])  # 8, 8, 19 splits
def test_consumers_take_partials_from_the_projection(rows, inner):
    """linear_partials -> add_rms_norm / qkv_norm_rope_cache equals the oracle
    chain bit for bit on integer inputs (the fold is exact there)."""
    g = gen(180 + rows + inner)
    hidden = 2560
    attended, wo = ints((rows, inner), -2, 2, g), ints((hidden, inner), -1, 1, g)
    residual = ints((rows, hidden), -8, 8, g)
    gain = normal((hidden,), 1.0, 0.1, g)
    parts = sk.linear_partials(attended.to(DEV), wo.to(DEV))
    total, normed = add_rms_norm(residual.to(DEV), parts, gain.to(DEV), 1e-6)
    ref_total, ref_normed = O.add_rms_norm(bits(residual), O.linear_partials(bits(attended), bits(wo), parts.shape[0]),
                                           bits(gain), 1e-6)
    assert_bits_exact(total, ref_total, what="total")
    assert_bits_exact(normed, ref_normed, what="normed")

    batch, nq, nk, d, capacity, k = 2, 32, 8, 128, 9, 2560
    x, wqkv = ints((batch, k), -2, 2, g), ints(((nq + 2 * nk) * d, k), -1, 1, g)
    qw, kw = normal((d,), 1.0, 0.1, g), normal((d,), 1.0, 0.1, g)
    cos, sin = normal((capacity, d), g=g), normal((capacity, d), g=g)
    parts = sk.linear_partials(x.to(DEV), wqkv.to(DEV))
    cache0 = torch.full((batch, nk, capacity, d), 33.0, dtype=torch.bfloat16)
    keys, values = cache0.to(DEV), cache0.to(DEV)
    q = qkv_norm_rope_cache(parts, qw.to(DEV), kw.to(DEV), 1e-6, 1e-6, cos.to(DEV), sin.to(DEV),
                            torch.tensor([5], device=DEV), keys, values)
    rq, rk, rv = O.qkv_norm_rope_cache(O.linear_partials(bits(x), bits(wqkv), parts.shape[0]),
                                       bits(qw), bits(kw), 1e-6, 1e-6, bits(cos), bits(sin), 5,
                                       bits(cache0), bits(cache0))
    assert_bits_exact(q, rq, what="q")
    assert_bits_exact(keys, rk, what="keys")
    assert_bits_exact(values, rv, what="values")


def test_graph_replay_follows_fresh_inputs():
    """tests/test_skinny_gemm.py:456-476 of the reference: both projections in
    one captured graph, replayed with new x and eager work in between."""
    g = gen(190)
    x = normal((4, 4096), g=g).to(DEV)
    w = (normal((2560, 4096), g=g) / 64).to(DEV)
    gate_up = (normal((2 * 2560, 4096), g=g) / 64).to(DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            sk.linear_partials(x, w)
            sk.linear_silu_mul(x, gate_up)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        partials = sk.linear_partials(x, w)
        hidden = sk.linear_silu_mul(x, gate_up)
    for seed in range(3):
        x.copy_(normal((4, 4096), g=gen(200 + seed)).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        eager = sk.linear_partials(x, w)
        assert torch.equal(partials, eager)
        assert_bits_exact(hidden, sk.linear_silu_mul(x, gate_up), what="graph silu")
        torch.testing.assert_close(partials.sum(0), F.linear(x.float(), w.float()), rtol=2e-3, atol=2e-3)
