"""Pin the CPU oracle (oracle/qf_oracle.c) before trusting it.

Each oracle function is checked against (a) the third-party arithmetic the
reference calls - transformers ``Qwen3RMSNorm``, ``apply_rotary_pos_emb``,
``Qwen3RotaryEmbedding`` and torch ``F.silu`` / ``F.embedding`` evaluated on
the CPU, (b) the committed golden fixtures in tests/golden, (c) the known
answers the reference's own tests use (constant rows with eps 0 are exact,
zeros stay zero, position 0 is the identity, split-K partials fold to the
same bits as their bf16 sum), and (d) planted mistakes that must be caught.
No GPU is used.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.nn import functional as F
from transformers import Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import (
    Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb)

from conftest import O, assert_bf16_close, bits, gen, normal

THETA = 5_000_000


def hf_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    m = Qwen3RMSNorm(x.shape[-1], eps=eps).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(w)
    with torch.inference_mode():
        return m(x)


def hf_rotary(positions: torch.Tensor, dim: int = 128):
    cfg = Qwen3Config(head_dim=dim, rope_theta=THETA, max_position_embeddings=32768,
                      hidden_size=256, num_attention_heads=2, num_key_value_heads=1)
    rot = Qwen3RotaryEmbedding(cfg)
    with torch.inference_mode():
        cos, sin = rot(torch.empty(0, dtype=torch.bfloat16), positions.view(1, -1))
    return cos[0], sin[0], rot.inv_freq


# ---------------------------------------------------------------- bf16 basics

def test_bf16_rounding_matches_torch():
    g = gen(1)
    f = torch.randn(200_000, generator=g) * torch.exp(torch.randn(200_000, generator=g) * 8)
    special = torch.tensor([0.0, -0.0, 1.0, -1.0, float("inf"), -float("inf"), float("nan"),
                            1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9,
                            3.4e38, 1e-40, -1e-45, 1.17549435e-38, 65504.0, 2.0 ** -133])
    f = torch.cat([f, special])
    expected = f.to(torch.bfloat16).view(torch.uint16).numpy()
    got = O.bf16_bits(f.numpy())
    # NaN bit patterns are not part of the contract (torch's vectorised CPU
    # cast gives 0xFFFF, its scalar c10::BFloat16 path 0x7FC0): compare NaN-ness.
    nan = np.isnan(f.numpy())
    assert np.array_equal(np.isnan(O.bf16_value(got)), nan)
    assert np.array_equal(got[~nan], expected[~nan])
    got_c = np.array([O.lib().or_bf16(float(v)) for v in special.numpy()], dtype=np.uint16)
    assert np.array_equal(got_c, got[-len(special):])


def test_ulp_distance():
    a = np.array([0x3F80, 0x3F80, 0x8000, 0x0000, 0xBF80, 0x0001], dtype=np.uint16)
    b = np.array([0x3F80, 0x3F81, 0x0000, 0x8001, 0xBF81, 0x8001], dtype=np.uint16)
    assert O.ulp_distance(a, b).tolist() == [0, 1, 0, 1, 1, 2]


# -------------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("rows,cols", [(8, 2560), (64, 2560), (33, 128), (5, 256), (3, 48)])
def test_rms_norm_matches_qwen3rmsnorm(rows, cols):
    g = gen(0)
    x = normal((rows, cols), g=g)
    w = normal((cols,), 1.0, 0.1, g=g)
    got = O.rms_norm(bits(x), bits(w), 1e-6)
    assert_bf16_close(got, hf_norm(x, w, 1e-6), max_ulp=1, min_exact=0.99, what="rms_norm")


def test_rms_norm_config1_golden(golden):
    d = golden["config1_rms_norm"]
    got = O.rms_norm(d["x"], d["w"], float(d["eps"]))
    assert_bf16_close(got, d["out"], max_ulp=1, min_exact=0.99, what="config 1 golden")


def test_rms_norm_known_answers():
    g = gen(2)
    w = normal((2560,), 1.0, 0.1, g=g)
    for c in (1.0, 2.0, 0.5, -4.0, 0.25):
        x = torch.full((3, 2560), c, dtype=torch.bfloat16)
        out = O.rms_norm(bits(x), bits(w), 0.0)
        expected = bits(torch.sign(torch.tensor(c)).to(torch.bfloat16) * w)
        assert np.array_equal(out, np.broadcast_to(expected, out.shape)), c
    zeros = O.rms_norm(np.zeros((2, 128), np.uint16), bits(w[:128]), 1e-6)
    assert not O.bf16_value(zeros).any()


def test_rms_norm_cast_placement_is_pinned():
    """Planted mistake: multiply the gain in f32 and round once.  The oracle
    must disagree with it while agreeing with Qwen3RMSNorm."""
    g = gen(3)
    x = normal((64, 2560), g=g)
    w = normal((2560,), 1.0, 0.1, g=g)
    f = x.float()
    inv = torch.rsqrt(f.pow(2).mean(-1, keepdim=True) + 1e-6)
    wrong = (f * inv * w.float()).to(torch.bfloat16)
    got = O.rms_norm(bits(x), bits(w), 1e-6)
    assert (O.ulp_distance(got, bits(wrong)) > 0).mean() > 0.01
    assert_bf16_close(got, hf_norm(x, w, 1e-6), max_ulp=1, min_exact=0.99)


# --------------------------------------------------------- add + RMSNorm

def test_add_rms_norm_bf16_branch():
    g = gen(4)
    r = normal((64, 2560), 0.0, 4.0, g=g)
    h = normal((64, 2560), g=g)
    w = normal((2560,), 1.0, 0.1, g=g)
    total, normed = O.add_rms_norm(bits(r), bits(h), bits(w), 1e-6)
    assert np.array_equal(total, bits(r + h))  # bf16 add is exact: atol 0
    assert_bf16_close(normed, hf_norm(r + h, w, 1e-6), max_ulp=1, min_exact=0.99)


def sum_partials_bf16(partials: torch.Tensor) -> torch.Tensor:
    """Sequential f32 sum then one bf16 rounding (tests/test_skinny_gemm.py:171-176)."""
    total = torch.zeros_like(partials[0])
    for p in partials:
        total = total + p
    return total.to(torch.bfloat16)


@pytest.mark.parametrize("splits", [1, 4, 8])
def test_add_rms_norm_split_k_folds_then_rounds_once(splits):
    g = gen(5)
    r = normal((7, 2560), g=g)
    partials = torch.randn((splits, 7, 2560), generator=g) * 0.5
    w = normal((2560,), 1.0, 0.1, g=g)
    direct = O.add_rms_norm(bits(r), bits(sum_partials_bf16(partials)), bits(w), 1e-6)
    folded = O.add_rms_norm(bits(r), partials.numpy(), bits(w), 1e-6)
    for a, b in zip(direct, folded):
        assert np.array_equal(a, b)
    # Planted mistake: rounding each partial to bf16 before the sum differs.
    if splits > 1:
        pre = sum_partials_bf16(partials.to(torch.bfloat16).float())
        wrong = O.add_rms_norm(bits(r), bits(pre), bits(w), 1e-6)
        assert not np.array_equal(wrong[0], folded[0])


# ---------------------------------------------------------------- SiLU * up

def test_silu_mul_matches_torch():
    g = gen(6)
    gu = normal((64, 2 * 9728), 0.0, 4.0, g=g)
    gu[0, :8] = torch.tensor([-40.0, -12.0, -1.0, 0.0, 1.0, 12.0, 40.0, 88.0])
    gate, up = gu.chunk(2, dim=-1)
    expected = F.silu(gate) * up
    got = O.silu_mul(bits(gu))
    assert_bf16_close(got, expected, max_ulp=1, min_exact=0.999, what="silu_mul")


def test_silu_mul_f64_bound_and_special_values():
    vals = torch.tensor([-100.0, -89.0, -88.0, -40.0, -12.0, -1.0, -0.0, 0.0, 1e-30, 1.0, 12.0,
                         40.0, 88.0, 1e30], dtype=torch.float32).to(torch.bfloat16)
    up = torch.ones_like(vals)
    got = O.bf16_value(O.silu_mul(bits(torch.cat([vals, up]).view(1, -1))))[0]
    g64 = vals.double().numpy()
    with np.errstate(over="ignore"):
        exact = g64 / (1.0 + np.exp(-g64))
    ref = O.bf16_value(O.bf16_bits(exact.astype(np.float32)))
    # f32 overflow of exp(-g) for g < -88.7 makes the reference exactly -0.
    exact_f32_path = np.where(g64 < -88.72, -0.0, ref)
    np.testing.assert_array_equal(got, exact_f32_path)
    # Planted mistake: no bf16 rounding of SiLU before the product.
    g = gen(7)
    gu = normal((16, 2 * 512), 0.0, 4.0, g=g)
    gate, upv = gu.float().chunk(2, dim=-1)
    wrong = (F.silu(gate) * upv).to(torch.bfloat16)
    assert (O.ulp_distance(O.silu_mul(bits(gu)), bits(wrong)) > 0).any()


# ---------------------------------------------------------- rotary tables

def test_default_inv_freq_matches_transformers():
    # Tables are built from the model's own inv_freq buffer; this helper only
    # has to agree with it to the accuracy of torch's f32 pow (about 1 ulp).
    _, _, inv = hf_rotary(torch.arange(2))
    np.testing.assert_array_max_ulp(O.default_inv_freq(THETA, 128), inv.numpy(), maxulp=2)


def test_rope_table_matches_qwen3_rotary_embedding():
    positions = torch.cat([torch.arange(2048), torch.tensor([4095, 8191, 16383, 32767])])
    cos, sin, inv = hf_rotary(positions)
    oc, os_ = O.rope_table(inv.numpy(), positions=positions.numpy())
    assert_bf16_close(oc, cos, max_ulp=1, min_exact=0.999, what="cos")
    assert_bf16_close(os_, sin, max_ulp=1, min_exact=0.999, what="sin")
    # Row 0 is the identity rotation.
    assert np.all(O.bf16_value(oc[0]) == 1.0) and np.all(O.bf16_value(os_[0]) == 0.0)
    # Implicit-slot form equals the explicit one.
    ic, is_ = O.rope_table(inv.numpy(), n_pos=2048)
    assert np.array_equal(ic, oc[:2048]) and np.array_equal(is_, os_[:2048])


def test_rope_table_golden(golden):
    d = golden["rope_table"]
    oc, os_ = O.rope_table(d["inv_freq"], positions=d["positions"])
    assert_bf16_close(oc, d["cos"], max_ulp=1, min_exact=0.99)
    assert_bf16_close(os_, d["sin"], max_ulp=1, min_exact=0.99)


# ------------------------------------------------------------ QK norm + RoPE

def hf_qk(q, k, qw, kw, cos, sin, q_eps, k_eps):
    """Qwen3RMSNorm + apply_rotary_pos_emb on [B, H, 1, 128] (the reference test)."""
    return apply_rotary_pos_emb(hf_norm(q, qw, q_eps), hf_norm(k, kw, k_eps), cos, sin)


@pytest.mark.parametrize("batch,shared", [(1, True), (3, False), (16, False), (4, True)])
def test_qk_norm_rope_matches_transformers(batch, shared):
    g = gen(8)
    q = normal((batch, 32, 1, 128), g=g)
    k = normal((batch, 8, 1, 128), g=g)
    qw, kw = normal((128,), 1.0, 0.1, g=g), normal((128,), 1.0, 0.1, g=g)
    pos = torch.randint(0, 32768, (1 if shared else batch,), generator=g)
    cos, sin, _ = hf_rotary(pos)
    cos, sin = cos.view(-1, 1, 128), sin.view(-1, 1, 128)
    eq, ek = hf_qk(q, k, qw, kw, cos, sin, 1e-6, 3e-6)
    oq, ok = O.qk_norm_rope(bits(q)[:, :, 0], bits(k)[:, :, 0], bits(qw), bits(kw), bits(cos),
                            bits(sin), 1e-6, 3e-6)
    assert_bf16_close(oq, bits(eq)[:, :, 0], max_ulp=1, min_exact=0.99, what="q")
    assert_bf16_close(ok, bits(ek)[:, :, 0], max_ulp=1, min_exact=0.99, what="k")


def test_qk_norm_rope_known_answers():
    """tests/test_qk_norm_rope.py:163-175 of the reference: exact normalisation
    (eps 0, constant rows) leaves only RoPE rounding, which must be bit-exact;
    zeros give zeros; position 0 is the identity after norm and gain."""
    g = gen(9)
    q = torch.ones(3, 32, 1, 128, dtype=torch.bfloat16)
    k = torch.full((3, 8, 1, 128), 2.0, dtype=torch.bfloat16)
    qw, kw = normal((128,), g=g), normal((128,), g=g)
    cos, sin, _ = hf_rotary(8191 + torch.arange(3))
    cos, sin = cos.view(3, 1, 128), sin.view(3, 1, 128)
    eq, ek = apply_rotary_pos_emb(q * qw, (k / 2) * kw, cos, sin)
    oq, ok = O.qk_norm_rope(bits(q)[:, :, 0], bits(k)[:, :, 0], bits(qw), bits(kw), bits(cos),
                            bits(sin), 0.0, 0.0)
    assert np.array_equal(oq, bits(eq)[:, :, 0]) and np.array_equal(ok, bits(ek)[:, :, 0])
    zq, zk = O.qk_norm_rope(np.zeros((3, 32, 128), np.uint16), np.zeros((3, 8, 128), np.uint16),
                            bits(qw), bits(kw), bits(cos), bits(sin), 1e-6, 1e-6)
    assert not O.bf16_value(zq).any() and not O.bf16_value(zk).any()
    # position 0: cos = 1, sin = 0 -> out = bf16(n * 1) + bf16(rot * 0) = n
    x = normal((2, 32, 1, 128), g=g)
    c0, s0, _ = hf_rotary(torch.zeros(1, dtype=torch.int64))
    oq, _ = O.qk_norm_rope(bits(x)[:, :, 0], bits(x)[:, :8, 0], bits(qw), bits(kw), bits(c0),
                           bits(s0), 1e-6, 1e-6)
    n = O.rms_norm(bits(x)[:, :, 0], bits(qw), 1e-6)
    assert np.array_equal(O.bf16_value(oq), O.bf16_value(n))


def test_qk_norm_rope_product_rounding_negative_control():
    """tests/test_prefill.py:276-285 of the reference: dropping the bf16
    rounding of the two RoPE products must change bits."""
    g = gen(10)
    q, k = normal((4, 32, 128), g=g), normal((4, 8, 128), g=g)
    qw, kw = normal((128,), g=g), normal((128,), g=g)
    cos, sin, _ = hf_rotary(torch.tensor([17, 300, 2047, 9999]))
    args = (bits(q), bits(k), bits(qw), bits(kw), bits(cos), bits(sin), 1e-6, 1e-6)
    right, wrong = O.qk_norm_rope(*args), O.qk_norm_rope(*args, round_products=False)
    assert any(not np.array_equal(a, b) for a, b in zip(right, wrong))


def test_qk_norm_rope_golden(golden):
    d = golden["qk_norm_rope"]
    oq, ok = O.qk_norm_rope(d["q"], d["k"], d["qw"], d["kw"], d["cos"], d["sin"],
                            float(d["q_eps"]), float(d["k_eps"]))
    assert_bf16_close(oq, d["oq"], max_ulp=1, min_exact=0.99)
    assert_bf16_close(ok, d["ok"], max_ulp=1, min_exact=0.99)


# ----------------------------------------------------- packed decode / prefill

def ref_qkv_norm_rope_cache(qkv, qw, kw, q_eps, k_eps, cos, sin, position, key_cache, value_cache):
    """Restates tests/test_decode_step.py:71-81 of the reference on CPU."""
    batch, kv_heads, _, width = key_cache.shape
    heads = qkv.shape[1] // width - 2 * kv_heads
    q, k, v = qkv.split([heads * width, kv_heads * width, kv_heads * width], dim=-1)
    q = hf_norm(q.reshape(batch, heads, 1, width), qw, q_eps)
    k = hf_norm(k.reshape(batch, kv_heads, 1, width), kw, k_eps)
    c, s = cos.index_select(0, position).unsqueeze(0), sin.index_select(0, position).unsqueeze(0)
    q, k = apply_rotary_pos_emb(q, k, c, s)
    key_cache.index_copy_(2, position, k)
    value_cache.index_copy_(2, position, v.reshape(batch, kv_heads, 1, width))
    return q.contiguous()


@pytest.mark.parametrize("batch,heads,kv,capacity", [(3, 32, 8, 640), (2, 4, 2, 129)])
def test_qkv_norm_rope_cache_oracle(batch, heads, kv, capacity):
    g = gen(11)
    cos, sin, _ = hf_rotary(torch.arange(capacity))
    qw, kw = normal((128,), g=g), normal((128,), g=g)
    for position in (0, capacity // 2, capacity - 1):
        qkv = normal((batch, (heads + 2 * kv) * 128), g=g)
        keys = torch.full((batch, kv, capacity, 128), float("nan"), dtype=torch.bfloat16)
        values = keys.clone()
        pos = torch.tensor([position])
        eq = ref_qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 3e-6, cos, sin, pos, keys, values)
        oq, ok_, ov = O.qkv_norm_rope_cache(bits(qkv), bits(qw), bits(kw), 1e-6, 3e-6, bits(cos),
                                            bits(sin), position,
                                            np.full(keys.shape, 0x7FC0, np.uint16),
                                            np.full(keys.shape, 0x7FC0, np.uint16))
        assert_bf16_close(oq, eq, max_ulp=1, min_exact=0.99)
        assert_bf16_close(ok_[:, :, position], keys[:, :, position], max_ulp=1, min_exact=0.99)
        assert np.array_equal(ov[:, :, position], bits(values[:, :, position]))
        untouched = np.arange(capacity) != position
        assert np.all(ok_[:, :, untouched] == 0x7FC0) and np.all(ov[:, :, untouched] == 0x7FC0)


def test_qkv_split_k_partials_equal_their_bf16_sum():
    """tests/test_skinny_gemm.py:283-317 of the reference, on the oracle."""
    g = gen(12)
    batch, nq, nk, cap, splits = 2, 4, 2, 5, 4
    partials = torch.randn((splits, batch, (nq + 2 * nk) * 128), generator=g) * 0.5
    qw, kw = normal((128,), g=g), normal((128,), g=g)
    cos, sin = normal((cap, 128), g=g), normal((cap, 128), g=g)
    cache = np.full((batch, nk, cap, 128), bits(torch.tensor(33.0, dtype=torch.bfloat16)))
    a = O.qkv_norm_rope_cache(bits(sum_partials_bf16(partials)), bits(qw), bits(kw), 1e-6, 1e-6,
                              bits(cos), bits(sin), 3, cache, cache)
    b = O.qkv_norm_rope_cache(partials.numpy(), bits(qw), bits(kw), 1e-6, 1e-6, bits(cos),
                              bits(sin), 3, cache, cache)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    v_expected = bits(sum_partials_bf16(partials))[:, (nq + nk) * 128:].reshape(batch, nk, 128)
    assert np.array_equal(b[2][:, :, 3], v_expected)


def test_qkv_out_of_range_position_guard():
    g = gen(13)
    qkv = normal((2, 48 * 128), g=g)
    qw, kw = normal((128,), g=g), normal((128,), g=g)
    cos, sin, _ = hf_rotary(torch.arange(16))
    cache = np.zeros((2, 8, 16, 128), np.uint16)
    for bad in (-1, 16, 10 ** 9):
        q, k, v = O.qkv_norm_rope_cache(bits(qkv), bits(qw), bits(kw), 1e-6, 1e-6, bits(cos),
                                        bits(sin), bad, cache, cache)
        assert np.all(q == 0x7FC0) and not k.any() and not v.any()


def reference_qkv(p, qw, kw, qe, ke, cos, sin, keys, values, length):
    """Restates tests/test_prefill.py:72-84 of the reference on CPU."""
    b, nk, _, d = keys.shape
    nq = p.shape[-1] // d - 2 * nk
    q, k, v = p.reshape(b, length, -1).split((nq * d, nk * d, nk * d), -1)
    q = hf_norm(q.reshape(b, length, nq, d), qw, qe)
    k = hf_norm(k.reshape(b, length, nk, d), kw, ke)

    def rotate(x):
        half = torch.cat((-x[..., d // 2:], x[..., :d // 2]), -1)
        return x * cos[None, :length, None, :] + half * sin[None, :length, None, :]

    q, k = rotate(q), rotate(k)
    keys[:, :, :length].copy_(k.transpose(1, 2))
    values[:, :, :length].copy_(v.reshape(b, length, nk, d).transpose(1, 2))
    return q.contiguous()


@pytest.mark.parametrize("b,t,c,nq,nk", [(1, 1, 3, 4, 2), (2, 7, 13, 4, 2), (1, 33, 39, 32, 8),
                                         (3, 3, 11, 6, 2), (2, 5, 9, 12, 4)])
def test_prefill_qkv_oracle(b, t, c, nq, nk):
    """Shapes of tests/test_prefill.py:235-238 of the reference."""
    g = gen(14)
    p = normal((b * t, (nq + 2 * nk) * 128), g=g)
    qw, kw = normal((128,), g=g), normal((128,), g=g)
    cos, sin, _ = hf_rotary(torch.arange(c))
    k = torch.full((b, nk, c, 128), float("nan"), dtype=torch.bfloat16)
    v = k.clone()
    eq = reference_qkv(p, qw, kw, 1e-6, 3e-6, cos, sin, k, v, t)
    oq, ok_, ov = O.prefill_qkv(bits(p), bits(qw), bits(kw), 1e-6, 3e-6, bits(cos), bits(sin),
                                np.full(k.shape, 0x7FC0, np.uint16),
                                np.full(k.shape, 0x7FC0, np.uint16), t)
    assert_bf16_close(oq, eq, max_ulp=1, min_exact=0.99)
    assert_bf16_close(ok_, k, max_ulp=1, min_exact=0.99)
    assert np.array_equal(ov, bits(v))


# ---------------------------------------------------------------- embedding

def test_embedding_bit_exact_and_guard():
    g = gen(15)
    table = normal((1000, 2560), 0.0, 0.02, g=g)
    ids = torch.randint(0, 1000, (4, 33), generator=g)
    assert np.array_equal(O.embedding(ids.numpy(), bits(table)), bits(F.embedding(ids, table)))
    bad = O.embedding(np.array([-1, 1000, 5]), bits(table))
    assert not bad[:2].any() and np.array_equal(bad[2], bits(table[5]))


def test_silu_mul_golden(golden):
    d = golden["silu_mul"]
    assert_bf16_close(O.silu_mul(d["gate_up"]), d["out"], max_ulp=1, min_exact=0.99)


def test_embedding_golden(golden):
    d = golden["embedding"]
    assert np.array_equal(O.embedding(d["ids"], d["table"]), d["out"])


# ------------------------------------------------------- decode projections

def _ints(shape, lo, hi, g):
    return torch.randint(lo, hi + 1, shape, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("m,n,k,splits", [(1, 32, 64, 1), (3, 64, 256, 4), (16, 96, 192, 3),
                                          (17, 32, 128, 2), (64, 64, 640, 10)])
def test_linear_partials_integer_known_answer(m, n, k, splits):
    # Small integers: every partial sum is an exact f32, so the oracle must equal
    # an int64 matmul of each K chunk bit for bit (pins indexing and the split).
    g = gen(40)
    x, w = _ints((m, k), -4, 4, g), _ints((n, k), -4, 4, g)
    got = O.linear_partials(bits(x), bits(w), splits)
    xi, wi = x.to(torch.int64), w.to(torch.int64)
    per = k // splits
    for s in range(splits):
        chunk = slice(s * per, (s + 1) * per)
        np.testing.assert_array_equal(got[s], (xi[:, chunk] @ wi[:, chunk].T).numpy().astype(np.float32))


def test_linear_partials_match_torch_float64():
    g = gen(41)
    x, w = normal((5, 512), g=g), normal((64, 512), 0.0, 0.05, g)
    got = O.linear_partials(bits(x), bits(w), 4)
    for s in range(4):
        chunk = slice(128 * s, 128 * (s + 1))
        exact = F.linear(x[:, chunk].double(), w[:, chunk].double()).float().numpy()
        np.testing.assert_array_equal(got[s], exact)  # exactly rounded, like float64 -> f32
    # the consumer's sum equals the full-K product up to f32 summation error
    full = F.linear(x.double(), w.double()).numpy()
    scale = (x.double().abs() @ w.double().abs().T).numpy()
    assert (np.abs(got.astype(np.float64).sum(0) - full) <= 4 * 2.0**-24 * scale + 1e-30).all()


def test_linear_partials_planted_mistakes_are_caught():
    g = gen(42)
    x, w = normal((4, 256), g=g), normal((32, 256), g=g)
    good = O.linear_partials(bits(x), bits(w), 2)
    exact = F.linear(x.double(), w.double()).numpy()
    # a dropped last 32-wide k step
    dropped = F.linear(x[:, :-32].double(), w[:, :-32].double()).numpy()
    # mismatched fragment layouts: x's k-group 8g..8g+7 against W's k-group g^1
    perm = torch.arange(256) ^ 8
    swapped = x.double() @ w.double()[:, perm].T
    total = good.astype(np.float64).sum(0)
    tol = 1e-4 * np.abs(exact).max()
    assert np.abs(total - exact).max() <= tol
    assert np.abs(dropped - exact).max() > tol
    assert np.abs(swapped.numpy() - exact).max() > tol


@pytest.mark.parametrize("m,n,k", [(1, 32, 128), (4, 64, 256), (16, 32, 640), (33, 32, 64)])
def test_linear_silu_mul_is_rounded_projections_then_silu_mul(m, n, k):
    g = gen(43)
    x = normal((m, k), 0.0, 2.0, g)
    gate_up = normal((2 * n, k), 0.0, 4.0 / k**0.5, g)
    got = O.linear_silu_mul(bits(x), bits(gate_up))
    # bf16 projections, exactly rounded (float64 -> f32 -> bf16), then SiLU * up
    proj = F.linear(x.double(), gate_up.double()).float().to(torch.bfloat16)
    np.testing.assert_array_equal(got, O.silu_mul(bits(proj)))
    # third-party arithmetic: torch F.silu on the bf16 projections
    gate, up = proj.chunk(2, dim=-1)
    assert_bf16_close(got, F.silu(gate) * up, max_ulp=1, min_exact=0.99, what="linear_silu_mul")


def test_linear_silu_mul_integer_known_answer_and_negative_control():
    g = gen(44)
    x, gate_up = _ints((8, 192), -2, 2, g), _ints((64, 192), -1, 1, g)
    got = O.linear_silu_mul(bits(x), bits(gate_up))
    proj = (x.to(torch.int64) @ gate_up.to(torch.int64).T).float().to(torch.bfloat16)
    np.testing.assert_array_equal(got, O.silu_mul(bits(proj)))
    # The reference's negative control: skipping the bf16 rounding of the
    # projections is a different function (tests/test_skinny_gemm.py:195-200).
    x = normal((64, 256), 0.0, 3.0, gen(45))
    w = normal((128, 256), g=gen(46))
    gate, up = F.linear(x.float(), w.float()).chunk(2, dim=-1)
    unrounded = (F.silu(gate) * up).to(torch.bfloat16)
    assert (O.ulp_distance(O.linear_silu_mul(bits(x), bits(w)), bits(unrounded)) > 0).any()


# --------------------------------------------------------- decode attention

def sdpa64(q, k, v, used):
    """torch float64 scaled_dot_product_attention per (sequence, kv head)."""
    batch, hq = q.shape[:2]
    hk = k.shape[1]
    g = hq // hk
    out = torch.zeros((batch, 1, hq, 128), dtype=torch.float64)
    for b in range(batch):
        for h in range(hk):
            n = int(used[b * hk + h])
            if n:
                out[b, 0, h * g:(h + 1) * g] = F.scaled_dot_product_attention(
                    q[b, h * g:(h + 1) * g, 0].double()[None], k[b, h, :n].double()[None],
                    v[b, h, :n].double()[None], scale=128 ** -0.5)[0]
    return out


@pytest.mark.parametrize("b,hq,hk,cap", [(1, 4, 1, 1), (1, 4, 1, 65), (2, 6, 2, 257), (3, 8, 2, 129),
                                         (1, 32, 8, 544), (1, 16, 1, 193)])
def test_decode_attention_matches_torch_float64(b, hq, hk, cap):
    g = gen(300 + cap)
    q, k, v = normal((b, hq, 1, 128), g=g), normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    used = (torch.arange(b * hk, dtype=torch.int32) * 37 % (cap + 1)).clamp(min=1)
    used[0] = cap
    poisoned_k, poisoned_v = k.clone(), v.clone()
    for vh in range(b * hk):
        poisoned_k.view(b * hk, cap, 128)[vh, int(used[vh]):] = float("nan")
        poisoned_v.view(b * hk, cap, 128)[vh, int(used[vh]):] = float("nan")
    got = O.decode_attention(bits(q), bits(poisoned_k), bits(poisoned_v), used.numpy(), 128 ** -0.5)
    assert not np.isnan(O.bf16_value(got)).any()  # slots past `used` are never read
    expected = sdpa64(q, k, v, used).to(torch.bfloat16)
    assert_bf16_close(got, expected, max_ulp=1, min_exact=0.999, what="decode attention")


def test_decode_attention_known_answers_and_planted_mistakes():
    # zero queries: uniform weights, so the output is the mean of the valid V rows
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 193, 128, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    v[:, :, :64], v[:, :, 64:128], v[:, :, 128:] = 2, 6, 20
    used = np.array([193], dtype=np.int32)
    got = O.bf16_value(O.decode_attention(bits(q), bits(k), bits(v), used, 128 ** -0.5))
    mean = (64 * 2 + 64 * 6 + 65 * 20) / 193
    assert (got == O.bf16_value(O.bf16_bits(np.float32(mean)))).all()
    assert not np.allclose(got, (2 + 6 + 20 + 20) / 4)  # equal segment weights would be wrong
    # one dominant block: all weight on the keys whose scores are largest
    q.fill_(32)
    k[:, :, :64], k[:, :, 64:128], k[:, :, 128:] = -32, 0, 32
    got = O.bf16_value(O.decode_attention(bits(q), bits(k), bits(v), used, 128 ** -0.5))
    assert (got == 20).all()
    # no valid key -> zeros
    got = O.decode_attention(bits(q), bits(k), bits(v), np.array([0], dtype=np.int32), 128 ** -0.5)
    assert (got == 0).all()
    # planted mistakes: the wrong kv head for a query head, or reading past `used`
    g = gen(310)
    q, k, v = normal((1, 8, 1, 128), g=g), normal((1, 2, 64, 128), g=g), normal((1, 2, 64, 128), g=g)
    used = torch.tensor([40, 64], dtype=torch.int32)
    good = O.decode_attention(bits(q), bits(k), bits(v), used.numpy(), 128 ** -0.5)
    swapped = sdpa64(q, k.flip(1), v.flip(1), used.flip(0)).to(torch.bfloat16)
    assert (O.ulp_distance(good, bits(swapped)) > 1).any()
    past_end = sdpa64(q, k, v, torch.tensor([64, 64], dtype=torch.int32)).to(torch.bfloat16)
    assert (O.ulp_distance(good, bits(past_end)) > 1).any()


# ------------------------------------------------ causal prefill attention

def causal64(q, k, v, length):
    """torch float64 scaled_dot_product_attention, is_causal, grouped heads:
    q [B, T, Hq, 128], k/v [B, Hkv, C, 128] -> [B, T, Hq, 128]."""
    hq, hk = q.shape[2], k.shape[1]
    kk = k[:, :, :length].double().repeat_interleave(hq // hk, 1)
    vv = v[:, :, :length].double().repeat_interleave(hq // hk, 1)
    out = F.scaled_dot_product_attention(q.double().transpose(1, 2), kk, vv, is_causal=True,
                                         scale=128 ** -0.5)
    return out.transpose(1, 2)


@pytest.mark.parametrize("b,t,hq,hk,cap", [(1, 1, 4, 2, 1), (2, 37, 8, 2, 40), (1, 70, 4, 4, 96),
                                           (1, 130, 8, 1, 130)])
def test_prefill_attention_matches_torch_float64(b, t, hq, hk, cap):
    g = gen(700 + t)
    q = normal((b, t, hq, 128), g=g)
    k, v = normal((b, hk, cap, 128), g=g), normal((b, hk, cap, 128), g=g)
    pk, pv = k.clone(), v.clone()
    pk[:, :, t:], pv[:, :, t:] = float("nan"), float("nan")   # slots past the prompt
    got = O.prefill_attention(bits(q), bits(pk), bits(pv), t, 128 ** -0.5)
    assert not np.isnan(O.bf16_value(got)).any()
    expected = causal64(q, k, v, t).to(torch.bfloat16)
    assert_bf16_close(got, expected, max_ulp=1, min_exact=0.999, what="prefill attention")


def test_prefill_attention_known_answers_and_planted_mistake():
    # zero queries: uniform weights over keys 0..t, the running mean of V
    t = 9
    q = torch.zeros(1, t, 4, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, t, 128, dtype=torch.bfloat16)
    v = torch.arange(t, dtype=torch.float32).view(1, 1, t, 1).expand(1, 2, t, 128).to(torch.bfloat16)
    got = O.bf16_value(O.prefill_attention(bits(q), bits(k), bits(v), t, 128 ** -0.5))
    for pos in range(t):
        assert (got[0, pos] == np.float32(pos / 2)).all()       # mean of 0..pos
    # one dominant key j0: every position from j0 on returns V[j0]
    q.fill_(8)
    k.fill_(-8)
    k[:, :, 4] = 8
    got = O.bf16_value(O.prefill_attention(bits(q), bits(k), bits(v), t, 128 ** -0.5))
    assert (got[0, 4:] == 4).all() and (got[0, 3] != 4).all()
    # planted mistake: attending one key past the diagonal
    g = gen(720)
    q, k, v = normal((1, 16, 4, 128), g=g), normal((1, 2, 17, 128), g=g), normal((1, 2, 17, 128), g=g)
    good = O.prefill_attention(bits(q), bits(k), bits(v), 16, 128 ** -0.5)
    hq, hk = 4, 2
    kk, vv = (x[:, :, :17].double().repeat_interleave(hq // hk, 1) for x in (k, v))
    mask = torch.ones(16, 17, dtype=torch.bool).tril(diagonal=1)
    shifted = F.scaled_dot_product_attention(q.double().transpose(1, 2), kk, vv, attn_mask=mask,
                                             scale=128 ** -0.5).transpose(1, 2).to(torch.bfloat16)
    assert (O.ulp_distance(good, bits(shifted)) > 1).any()


# --------------------------------------------------- LM head + token choice

def test_lm_head_argmax_matches_torch_and_breaks_ties_low():
    g = gen(500)
    x, w = normal((3, 256), g=g), normal((1024, 256), 0.0, 0.1, g)
    tokens, logits = O.lm_head_argmax(bits(x), bits(w))
    expected = F.linear(x.double(), w.double()).float().to(torch.bfloat16)
    np.testing.assert_array_equal(logits, bits(expected))
    np.testing.assert_array_equal(tokens, expected.argmax(-1).numpy())
    # integer inputs: many exactly equal logits; the first maximum wins
    xi = torch.zeros(5, 64, dtype=torch.bfloat16)
    xi[:, 0] = 1
    xi[:, 1:3] = torch.randint(0, 2, (5, 2), generator=g).to(torch.bfloat16)
    wi = torch.randint(-1, 2, (512, 64), generator=g).to(torch.bfloat16)
    tokens, logits = O.lm_head_argmax(bits(xi), bits(wi))
    exact = (xi.to(torch.int64) @ wi.to(torch.int64).T)
    assert all(int((exact[r] == exact[r].max()).sum()) > 1 for r in range(5))  # ties present
    np.testing.assert_array_equal(tokens, np.argmax(exact.numpy(), axis=1))    # numpy: first maximum
    # planted mistake: the last maximum instead of the first
    last = exact.shape[1] - 1 - np.argmax(exact.numpy()[:, ::-1], axis=1)
    assert (tokens != last).any()
