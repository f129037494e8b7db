"""One-workgroup-per-CU decode projections (``kernels.row_gemv``) on the
MI355X against the CPU oracle.

Parity bar (the kernels accumulate each output over the whole K range in f32
with v_dot2c_f32_bf16, so only inputs whose sums are exact f32 values have
one right answer):

* integer-valued bf16 inputs: every sum is an exact f32 value, so ``y``,
  ``total`` (= ``add_rms_norm``'s total of the oracle) and the sums of
  squares must be bit-exact, at the Qwen3-4B shapes and at every row count;
* the RMSNorm prologue: with one-hot weight rows each output is one element
  of the normalised row, which must equal the oracle's ``add_rms_norm``
  output bit for bit (so the chain residual -> total -> normed reproduces
  the two-launch path exactly);
* random inputs: each output within half a bf16 ulp of the exact dot product
  plus 2^-16 * sum|x*w| (f32 accumulation error; a dropped chunk or a
  mismatched column is ~1/K of the magnitude, far above it), >= 99%
  bit-exact against the oracle's exactly rounded projection, and within the
  reference's own F.linear tolerance (tests/test_skinny_gemm.py:403-436).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import O, assert_bf16_close, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels import row_gemv as rg  # noqa: E402
from starter_amd.kernels.rotary import default_inv_freq, rope_tables  # noqa: E402
from starter_amd.kernels.small_query_attention import SmallQueryAttention  # noqa: E402

DEV = "cuda"
QWEN = {"down": (2560, 9728), "qkv": (6144, 2560), "o": (2560, 4096)}
CASES = [(rows, n, k) for rows in (1, 2, 3, 4) for n, k in
         [(2560, 9728), (6144, 2560), (2560, 4096), (512, 64), (8192, 256), (2048, 520)]
         if (rows if rows <= 2 else 4) * (n // 256) <= 128]


def ints(shape, lo, hi, g):
    return torch.randint(lo, hi + 1, shape, generator=g).to(torch.bfloat16)


TOL = 2.0**-16


def check_random(got, x, w, what):
    """got (bf16 [rows, n]) against x @ w.T: the f32-accumulation bound, and
    mostly bit-exact against the oracle's exactly rounded projection."""
    exact = x.double() @ w.double().T
    scale = x.double().abs() @ w.double().abs().T
    value = got.double().cpu()
    half_ulp = torch.ldexp(torch.ones_like(exact), torch.frexp(exact.abs().clamp_min(1e-30))[1] - 9)
    err = (value - exact).abs()
    assert bool((err <= half_ulp + TOL * scale + 1e-30).all()), (what, float((err - half_ulp).max()))
    want = bits(torch.from_numpy(O.linear_partials(bits(x), bits(w), 1)[0]).to(torch.bfloat16))
    exact_share = float((bits(got) == want).mean())
    assert exact_share >= 0.99, (what, exact_share)


def exact_bf16(x, w):
    """bf16 bits of x @ w.T for integer-valued operands (exact in f64 and f32)."""
    return bits((x.double() @ w.double().T).float().to(torch.bfloat16))


def group_squares(total_bits, groups=256):
    """f64 [rows, groups]: sums of squares of each group's consecutive columns."""
    v = O.bf16_value(total_bits).astype(np.float64)
    rows, n = v.shape
    return (v * v).reshape(rows, groups, n // groups).sum(-1)


@pytest.mark.parametrize("rows,n,k", CASES)
def test_rows_integer_exact(rows, n, k):
    g = gen(900 + rows + n + k)
    x, w = ints((rows, k), -3, 3, g), ints((n, k), -3, 3, g)
    got = rg.linear_rows(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    assert got.shape == (rows, n)
    assert_bits_exact(got, exact_bf16(x, w), f"rows={rows} n={n} k={k}")


@pytest.mark.parametrize("rows", [1, 2, 4])
@pytest.mark.parametrize("name", ["down", "qkv", "o"])
def test_rows_random_qwen_shapes(rows, name):
    n, k = QWEN[name]
    g = gen(950 + rows)
    x, w = normal((rows, k), g=g), normal((n, k), std=0.02, g=g)
    xd, wd = x.to(DEV), w.to(DEV)
    got = rg.linear_rows(xd, wd)
    check_random(got, x, w, f"{name} rows={rows}")
    torch.testing.assert_close(got, torch.nn.functional.linear(xd, wd), rtol=1.6e-2, atol=1e-2)
    for before, after in ((x, xd), (w, wd)):  # inputs untouched
        assert torch.equal(before.view(torch.int16), after.cpu().view(torch.int16))


@pytest.mark.parametrize("rows,n,k", [c for c in CASES if c[1] in (2560, 512, 2048)])
def test_residual_integer_exact(rows, n, k):
    """total = oracle add_rms_norm's total of y = x W^T; sq = exact group sums."""
    g = gen(1000 + rows + n)
    x, w = ints((rows, k), -2, 2, g), ints((n, k), -2, 2, g)
    residual = ints((rows, n), -50, 50, g)
    total, sq = rg.linear_residual(x.to(DEV), w.to(DEV), residual.to(DEV))
    torch.cuda.synchronize()
    want_total, _ = O.add_rms_norm(bits(residual), exact_bf16(x, w), np.ones(n, np.uint16), 1e-6)
    assert_bits_exact(total, want_total, f"total rows={rows} n={n}")
    assert sq.dtype == torch.float64 and sq.shape == (rows, 256)
    np.testing.assert_array_equal(sq.cpu().numpy(), group_squares(want_total))


def test_residual_in_place_and_random():
    """total may alias the residual; random inputs stay within an ulp of the
    oracle's total (y within an ulp, one more rounding)."""
    g = gen(1010)
    rows, (n, k) = 1, QWEN["down"]
    x, w, residual = normal((rows, k), g=g), normal((n, k), std=0.02, g=g), normal((rows, n), std=2, g=g)
    res_d = residual.to(DEV)
    total, sq = rg.linear_residual(x.to(DEV), w.to(DEV), res_d)
    y = bits(torch.from_numpy(O.linear_partials(bits(x), bits(w), 1)[0]).to(torch.bfloat16))
    want_total, _ = O.add_rms_norm(bits(residual), y, np.ones(n, np.uint16), 1e-6)
    assert_bf16_close(total, want_total, max_ulp=1, min_exact=0.99, what="total")
    np.testing.assert_allclose(sq.cpu().numpy(), group_squares(bits(total)), rtol=1e-14, atol=0)
    # the same call written into its own residual buffer gives the same bits
    from starter_amd.kernels import _lib
    sq2 = torch.empty_like(sq)
    _lib.call("qf_linear_residual", x.to(DEV).data_ptr(), rows, k, w.to(DEV).data_ptr(), n,
              res_d.data_ptr(), res_d.data_ptr(), sq2.data_ptr(), _lib.stream(res_d.device))
    torch.cuda.synchronize()
    assert torch.equal(res_d.view(torch.int16), total.view(torch.int16))
    assert torch.equal(sq2, sq)


def one_hot(n, k, g):
    """W [n, k] with a single 1 per row at column perm[r]; returns (W, perm)."""
    perm = torch.randint(0, k, (n,), generator=g)
    w = torch.zeros(n, k)
    w[torch.arange(n), perm] = 1.0
    return w.to(torch.bfloat16), perm.numpy()


@pytest.mark.parametrize("rows,heavy", [(1, False), (2, False), (3, False), (4, False),
                                        (1, True), (4, True)])
def test_normed_prologue_is_add_rms_norm_bit_for_bit(rows, heavy):
    """residual + y -> (total, sq) -> normed row, against the oracle's
    add_rms_norm(residual, y) normed output, element for element.  ``heavy``
    rows mimic Qwen3's massive activations: a few +-1e3..1e4 entries among
    +-1e-3 ones, so the squares span more exponent range than a double holds
    exactly and the per-workgroup sums are added in another order than the
    oracle's; the normalised rows still agree once the total is rounded to
    f32 (they could differ only where that rounding is a near tie)."""
    g = gen(1100 + rows + 50 * heavy)
    n_down, k_down = (2560, 512) if rows <= 2 else (2048, 512)
    x, wd = normal((rows, k_down), g=g), normal((n_down, k_down), std=0.05, g=g)
    residual = normal((rows, n_down), std=2.0, g=g)
    if heavy:
        x = x * 1e-3
        residual = (residual.float() * 1e-3).to(torch.bfloat16)
        spikes = torch.randint(0, n_down, (rows, 6), generator=g)
        magnitude = torch.exp(torch.empty(rows, 6).uniform_(6.9, 9.2, generator=g))
        sign = torch.randint(0, 2, (rows, 6), generator=g) * 2 - 1
        residual.scatter_(1, spikes, (magnitude * sign).to(torch.bfloat16))
    gain = normal((n_down,), mean=1.0, std=0.1, g=g)
    eps = 1e-6
    total, sq = rg.linear_residual(x.to(DEV), wd.to(DEV), residual.to(DEV))
    n_next = 256 * (8 if rows <= 2 else 4)
    w1, perm = one_hot(n_next, n_down, g)
    out = rg.linear_normed(total, sq, gain.to(DEV), eps, w1.to(DEV))
    torch.cuda.synchronize()
    if heavy:
        spread = O.bf16_value(bits(total)).astype(np.float64) ** 2
        spread = spread[spread > 0]
        assert np.log2(spread.max() / spread.min()) > 53 - 16   # beyond exact f64 sums
    # the oracle's RMSNorm of the same total (add_rms_norm's normalisation step)
    normed = O.rms_norm(bits(total), bits(gain), eps)
    assert_bits_exact(out, normed[:, perm], f"rows={rows} heavy={heavy}")


@pytest.mark.parametrize("rows", [1, 4])
def test_normed_random_qkv_shape(rows):
    n, k = (6144, 2560) if rows == 1 else (2048, 2560)
    g = gen(1200 + rows)
    total = normal((rows, k), std=3.0, g=g)
    gain = normal((k,), mean=1.0, std=0.1, g=g)
    w = normal((n, k), std=0.02, g=g)
    sq = torch.from_numpy(group_squares(bits(total)))
    out = rg.linear_normed(total.to(DEV), sq.to(DEV), gain.to(DEV), 1e-6, w.to(DEV))
    normed = torch.from_numpy(O.rms_norm(bits(total), bits(gain), 1e-6)).view(torch.bfloat16)
    check_random(out, normed, w, f"normed rows={rows}")


def sums_of_squares(total_bits, groups=256):
    """f64 [rows, groups] whose row sums are the exact sums of squares."""
    v = O.bf16_value(total_bits).astype(np.float64)
    sq = np.zeros((v.shape[0], groups))
    sq[:, 0] = (v * v).sum(-1)
    return torch.from_numpy(sq)


SILU_CASES = [(1, 9728, 2560), (1, 512, 256), (2, 1024, 512), (4, 512, 64), (3, 2048, 128)]


@pytest.mark.parametrize("rows,n,k", SILU_CASES)
def test_silu_normed_one_hot_exact(rows, n, k):
    """One-hot gate and up rows pick elements of the normalised row: the
    output must be the oracle's SiLU * up of exactly those elements."""
    g = gen(1400 + rows + n)
    total = normal((rows, k), std=2.0, g=g)
    gain = normal((k,), mean=1.0, std=0.1, g=g)
    w, perm = one_hot(2 * n, k, g)
    out = rg.linear_silu_mul_normed(total.to(DEV), sums_of_squares(bits(total)).to(DEV),
                                    gain.to(DEV), 1e-6, w.to(DEV))
    torch.cuda.synchronize()
    assert out.shape == (rows, n)
    normed = O.rms_norm(bits(total), bits(gain), 1e-6)
    want = O.silu_mul(np.concatenate([normed[:, perm[:n]], normed[:, perm[n:]]], axis=1))
    assert_bits_exact(out, want, f"rows={rows} n={n} k={k}")


@pytest.mark.parametrize("rows,n,k", SILU_CASES[:3])
def test_silu_normed_random(rows, n, k):
    g = gen(1450 + rows + n)
    total = normal((rows, k), std=2.0, g=g)
    gain = normal((k,), mean=1.0, std=0.1, g=g)
    w = normal((2 * n, k), std=0.05, g=g)
    out = rg.linear_silu_mul_normed(total.to(DEV), sums_of_squares(bits(total)).to(DEV),
                                    gain.to(DEV), 1e-6, w.to(DEV))
    normed = O.rms_norm(bits(total), bits(gain), 1e-6)
    want = O.linear_silu_mul(normed, bits(w))
    have_v, want_v = O.bf16_value(bits(out)), O.bf16_value(want)
    np.testing.assert_allclose(have_v, want_v, rtol=2e-2, atol=2e-2)
    assert float((bits(out) == want).mean()) >= 0.99


SCALE = 128 ** -0.5
MERGED_CASES = (  # b, hq, hk, cap, n, used rule
    (1, 32, 8, 545, 2560, "full"),     # Qwen3-4B batch 1: 9 segments
    (1, 32, 8, 1100, 2560, "full"),    # 18 segments: two batches in the merge
    (2, 32, 8, 700, 2560, "mixed"),
    (4, 8, 2, 300, 512, "mixed"),      # some heads attend nothing (zero rows)
    (3, 16, 1, 193, 1024, "full"),     # 16 query rows per kv head
)


@pytest.mark.parametrize("b,hq,hk,cap,n,rule", MERGED_CASES)
def test_residual_merged_equals_merge_then_residual(b, hq, hk, cap, n, rule):
    """o_proj over the unmerged attention segments with the residual add
    equals the attention's merged output through linear_residual, bit for bit."""
    g = gen(1500 + cap + b)
    qkv = (torch.randn((4, b, (hq + 2 * hk) * 128), generator=g) * 0.7).to(DEV)
    qw, kw = normal((128,), 1.0, 0.1, g).to(DEV), normal((128,), 1.0, 0.1, g).to(DEV)
    k, v = normal((b, hk, cap, 128), g=g).to(DEV), normal((b, hk, cap, 128), g=g).to(DEV)
    w = normal((n, hq * 128), 0.0, 0.02, g).to(DEV)
    residual = normal((b, n), std=2.0, g=g).to(DEV)
    if rule == "full":
        used = torch.full((b * hk,), cap, dtype=torch.int32)
    else:
        used = torch.arange(b * hk, dtype=torch.int32) * 97 % (cap + 1)
        used[-1] = 0
        used[0] = cap
    used = used.to(DEV)
    cos, sin = rope_tables(default_inv_freq(5_000_000.0, 128), cap, device=DEV)
    plan = SmallQueryAttention(b, hq, hk, cap, DEV)
    assert plan.splits > 1 and rg.supports_merged_shape(b, plan.splits, hq, hk, n)
    position = torch.tensor([cap - 1], dtype=torch.int64, device=DEV)
    k1, v1, k2, v2 = k.clone(), v.clone(), k.clone(), v.clone()
    with torch.inference_mode():
        attended = plan.run_qkv(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k1, v1, used, SCALE)
        want_total, want_sq = rg.linear_residual(attended.view(b, -1), w, residual)
        plan.partials.fill_(float("nan"))  # only what the second call writes may be read
        plan.stats.fill_(float("nan"))
        plan.run_qkv_unmerged(qkv, qw, kw, 1e-6, 2e-6, cos, sin, position, k2, v2, used, SCALE)
        total, sq = rg.linear_residual_merged(plan.partials, plan.stats, b, w, residual)
    torch.cuda.synchronize()
    assert_bits_exact(total, want_total, f"total (S={plan.splits})")
    assert torch.equal(sq, want_sq)
    assert_bits_exact(k2, k1, "key cache")


def test_graph_replay_follows_fresh_inputs():
    g = gen(1300)
    (n, k), (n2, k2) = QWEN["down"], QWEN["qkv"]
    x = normal((1, k), g=g).to(DEV)
    wd = normal((n, k), std=0.02, g=g).to(DEV)
    wq = normal((n2, k2), std=0.02, g=g).to(DEV)
    residual = normal((1, n), std=2.0, g=g).to(DEV)
    gain = normal((k2,), mean=1.0, std=0.1, g=g).to(DEV)

    def chain():
        total, sq = rg.linear_residual(x, wd, residual)
        return total, rg.linear_normed(total, sq, gain, 1e-6, wq)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        chain()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        total_g, out_g = chain()
    for seed in (1301, 1302, 1303):
        gg = gen(seed)
        x.copy_(normal((1, k), g=gg)); residual.copy_(normal((1, n), std=2.0, g=gg))
        graph.replay()
        torch.cuda.synchronize()
        total_e, out_e = chain()
        torch.cuda.synchronize()
        assert torch.equal(total_g.view(torch.int16), total_e.view(torch.int16))
        assert torch.equal(out_g.view(torch.int16), out_e.view(torch.int16))


def test_shape_rule():
    w = torch.zeros(2560, 9728, dtype=torch.bfloat16, device=DEV)
    assert rg.supports(torch.zeros(1, 9728, dtype=torch.bfloat16, device=DEV), w)
    assert not rg.supports(torch.zeros(5, 9728, dtype=torch.bfloat16, device=DEV), w)
    assert rg.supports(torch.zeros(3, 9728, dtype=torch.bfloat16, device=DEV), w)  # 4 x 10 outputs
    assert not rg.supports(torch.zeros(1, 9728, dtype=torch.bfloat16, device=DEV), w[:2304])  # 9 columns
    assert not rg.supports(torch.zeros(1, 9728, dtype=torch.float32, device=DEV), w)
    with pytest.raises(ValueError):
        rg.linear_rows(torch.zeros(1, 9720, dtype=torch.bfloat16, device=DEV), w[:, :9720])
