"""Host logic of the drop-in wrappers, on the CPU.

* Every wrapper rejects CPU tensors and malformed shapes with ``ValueError``
  before any launch (no fallback path exists).
* With fake CUDA tensor metadata (as tests/test_prefill.py:287-315 of the
  reference does for its Triton launch) the C-ABI receives the expected
  dimensions, strides, split counts and epsilons.
* The two-level row walk of ``rms_norm`` addresses exactly the rows of
  ``x.reshape(-1, C)`` for every layout it accepts without a copy.
"""

from __future__ import annotations

import math
from contextlib import contextmanager
from unittest import mock

import pytest
import torch

from starter_amd.kernels import _lib, decode_fused, embedding, prefill, qk_norm_rope, rmsnorm, rotary

BF16 = torch.bfloat16


class Fake:
    """Tensor metadata only: enough for the wrappers, never dereferenced."""

    _next = 0x100000

    def __init__(self, shape, dtype=BF16, strides=None, cuda=True, ptr=None):
        self.shape = torch.Size(shape)
        self.ndim = len(self.shape)
        self.dtype = dtype
        self.is_cuda = cuda
        self.device = torch.device("cuda", 0) if cuda else torch.device("cpu")
        self._strides = tuple(strides) if strides is not None else self._dense()
        if ptr is None:
            Fake._next += 1 << 20
            ptr = Fake._next
        self._ptr = ptr

    def _dense(self):
        out, acc = [], 1
        for size in reversed(self.shape):
            out.append(acc)
            acc *= size
        return tuple(reversed(out))

    def is_contiguous(self):
        dense = self._dense()
        return all(s == d for s, d, n in zip(self._strides, dense, self.shape) if n != 1)

    def contiguous(self):
        return self if self.is_contiguous() else Fake(self.shape, self.dtype, cuda=self.is_cuda)

    def stride(self, dim=None):
        return self._strides if dim is None else self._strides[dim]

    def data_ptr(self):
        return self._ptr

    def numel(self):
        return math.prod(self.shape)


@contextmanager
def recorded():
    calls = []
    fake_empty = lambda shape, *a, **k: Fake(shape, k.get("dtype", BF16))  # noqa: E731
    with mock.patch.object(_lib, "call", side_effect=lambda *a: calls.append(a)), \
            mock.patch.object(_lib, "stream", return_value=0), \
            mock.patch.object(torch, "empty", side_effect=fake_empty), \
            mock.patch.object(torch, "empty_like", side_effect=lambda t, **k: Fake(t.shape, t.dtype)):
        yield calls


# --------------------------------------------------------- CPU tensors rejected

def test_cpu_tensors_raise_value_error():
    x = torch.zeros(4, 2560, dtype=BF16)
    w = torch.zeros(2560, dtype=BF16)
    with pytest.raises(ValueError):
        rmsnorm.rms_norm(x, w, 1e-6)
    with pytest.raises(ValueError):
        decode_fused.add_rms_norm(x, x, w, 1e-6)
    with pytest.raises(ValueError):
        decode_fused.silu_mul(torch.zeros(4, 64, dtype=BF16))
    q, k = torch.zeros(2, 32, 1, 128, dtype=BF16), torch.zeros(2, 8, 1, 128, dtype=BF16)
    cs = torch.zeros(2, 1, 128, dtype=BF16)
    with pytest.raises(ValueError):
        qk_norm_rope.qk_norm_rope(q, k, w[:128], w[:128], cs, cs, 1e-6, 1e-6)
    keys = torch.zeros(2, 8, 16, 128, dtype=BF16)
    table = torch.zeros(16, 128, dtype=BF16)
    with pytest.raises(ValueError):
        decode_fused.qkv_norm_rope_cache(torch.zeros(2, 6144, dtype=BF16), w[:128], w[:128], 1e-6,
                                         1e-6, table, table, torch.zeros(1, dtype=torch.int64),
                                         keys, keys.clone())
    with pytest.raises(ValueError):
        prefill.prefill_qkv(torch.zeros(2 * 4, 6144, dtype=BF16), w[:128], w[:128], 1e-6, 1e-6,
                            table, table, keys, keys.clone(), 4)
    with pytest.raises(ValueError):
        embedding.embedding(torch.zeros(3, dtype=torch.int64), torch.zeros(10, 8, dtype=BF16))
    with pytest.raises(ValueError):
        rotary.rope_tables(rotary.default_inv_freq(5e6, 128), 16)


# ------------------------------------------------------------------ rms_norm

def test_rms_norm_limits_and_marshalling():
    w = Fake((2560,))
    with pytest.raises(ValueError):
        rmsnorm.rms_norm(Fake((4, 8193)), Fake((8193,)), 1e-6)
    with pytest.raises(ValueError):
        rmsnorm.rms_norm(Fake((4, 2560), torch.float32), w, 1e-6)
    with pytest.raises(ValueError):
        rmsnorm.rms_norm(Fake((4, 2560)), Fake((2561,)), 1e-6)
    with recorded() as calls:
        x = Fake((4, 2048, 2560))
        out = rmsnorm.rms_norm(x, w, 1e-6)
    assert tuple(out.shape) == (4, 2048, 2560)
    (name, src, rows, cols, inner, o_stride, i_stride, wp, eps, outp, stream), = calls
    assert (name, src, rows, cols, wp) == ("qf_rms_norm", x.data_ptr(), 8192, 2560, w.data_ptr())
    assert rows % inner == 0 and i_stride == 2560 and eps == 1e-6


@pytest.mark.parametrize("make", [
    lambda: torch.randn(4, 7, 48),
    lambda: torch.randn(4, 7, 48).transpose(0, 1),
    lambda: torch.randn(6, 96)[:, :48],
    lambda: torch.randn(3, 5, 2, 48)[:, :, 1],
    lambda: torch.randn(2, 3, 4, 48).permute(2, 0, 1, 3),
    lambda: torch.randn(1, 1, 48),
    lambda: torch.randn(48),
    lambda: torch.randn(5, 1, 3, 48).transpose(0, 2),
])
def test_row_walk_addresses_every_row(make):
    x = make()
    cols = x.shape[-1]
    rows, inner, o_stride, i_stride, src = rmsnorm._row_walk(x)
    flat = src.reshape(-1, cols)
    assert rows == flat.shape[0]
    storage = torch.as_strided(src, (src.untyped_storage().nbytes() // src.element_size(),), (1,),
                               0)
    base = src.storage_offset()
    for r in range(rows):
        start = base + (r // inner) * o_stride + (r % inner) * i_stride
        assert torch.equal(storage[start:start + cols], flat[r]), r


# ------------------------------------------------------------- add_rms_norm

def test_add_rms_norm_validation_and_splits():
    x, w = Fake((64, 2560)), Fake((2560,))
    with pytest.raises(ValueError):
        decode_fused.add_rms_norm(Fake((64, 2560), torch.float32), x, w, 1e-6)
    with pytest.raises(ValueError):
        decode_fused.add_rms_norm(x, Fake((64, 64)), w, 1e-6)
    with pytest.raises(ValueError):
        decode_fused.add_rms_norm(x, x, Fake((2048,)), 1e-6)
    with pytest.raises(ValueError):
        decode_fused.add_rms_norm(x, Fake((0, 64, 2560), torch.float32), w, 1e-6)
    with pytest.raises(ValueError):
        decode_fused.add_rms_norm(x, Fake((8, 64, 2560), torch.float32, cuda=False), w, 1e-6)
    with recorded() as calls:
        branch = Fake((8, 64, 2560), torch.float32)
        decode_fused.add_rms_norm(x, branch, w, 3e-6)
        decode_fused.add_rms_norm(x, x, w, 1e-6)
    (n0, *a0), (n1, *a1) = calls
    assert n0 == n1 == "qf_add_rms_norm"
    assert a0[:6] == [x.data_ptr(), branch.data_ptr(), 8, w.data_ptr(), 64, 2560]
    assert a0[6] == 3e-6 and a1[2] == 0


def test_silu_mul_validation_and_marshalling():
    with pytest.raises(ValueError):
        decode_fused.silu_mul(Fake((4, 19455)))
    with pytest.raises(ValueError):
        decode_fused.silu_mul(Fake((4, 19456), strides=(1, 4)))
    with recorded() as calls:
        out = decode_fused.silu_mul(Fake((8192, 19456)), block=512)
    assert tuple(out.shape) == (8192, 9728)
    (name, _, rows, cols, outp, _), = calls
    assert (name, rows, cols, outp) == ("qf_silu_mul", 8192, 9728, out.data_ptr())


# ------------------------------------------------------------ qk_norm_rope

def test_qk_norm_rope_strides_and_copies():
    qw, kw = Fake((128,)), Fake((128,))
    cs = Fake((3, 1, 128))
    with recorded() as calls:
        # the module path's view: [B, 1, H, D] projections transposed to [B, H, 1, D]
        q = Fake((3, 32, 1, 128), strides=(32 * 128, 128, 32 * 128, 1))
        k = Fake((3, 8, 1, 128), strides=(8 * 128, 128, 8 * 128, 1))
        qk_norm_rope.qk_norm_rope(q, k, qw, kw, cs, cs, 1e-6, 3e-6)
        # head rows 8 elements apart cannot use the 16-byte path: copied first
        qs = Fake((3, 32, 1, 128), strides=(40 * 128, 132, 128, 1))
        qk_norm_rope.qk_norm_rope(qs, k, qw, kw, Fake((1, 1, 128)), Fake((1, 1, 128)), 1e-6, 3e-6)
    (n0, *a0), (n1, *a1) = calls
    assert a0[:9] == [q.data_ptr(), k.data_ptr(), 3, 32, 8, 4096, 128, 1024, 128]
    assert a0[13] == 128 and (a0[14], a0[15]) == (1e-6, 3e-6)
    assert a1[0] != qs.data_ptr() and a1[5:7] == [4096, 128] and a1[13] == 0
    with pytest.raises(ValueError):
        qk_norm_rope.qk_norm_rope(Fake((3, 32, 2, 128)), k, qw, kw, cs, cs, 1e-6, 1e-6)
    with pytest.raises(ValueError):
        qk_norm_rope.qk_norm_rope(q, k, qw, kw, Fake((2, 1, 128)), Fake((2, 1, 128)), 1e-6, 1e-6)


# --------------------------------------------------- qkv_norm_rope_cache

def test_qkv_norm_rope_cache_contract():
    """Contract violations of tests/test_decode_step.py:325-334 of the reference."""
    qw, kw = Fake((128,)), Fake((128,))
    keys, values = Fake((3, 8, 640, 128)), Fake((3, 8, 640, 128))
    cos, sin = Fake((640, 128)), Fake((640, 128))
    pos = Fake((1,), torch.int64)
    qkv = Fake((3, 48 * 128))
    with recorded() as calls:
        q = decode_fused.qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 3e-6, cos, sin, pos, keys, values)
        partials = Fake((4, 3, 48 * 128), torch.float32)
        decode_fused.qkv_norm_rope_cache(partials, qw, kw, 1e-6, 3e-6, cos, sin, pos, keys, values)
    assert tuple(q.shape) == (3, 32, 1, 128)
    (n0, *a0), (n1, *a1) = calls
    assert a0[:5] == [qkv.data_ptr(), 0, 3, 32, 8] and a1[1] == 4
    assert a0[11:13] == [pos.data_ptr(), 640]
    bad = [
        (qkv, qw, kw, cos, sin, Fake((1,), torch.int32), keys, values),      # int32 position
        (Fake((3, 48 * 128 - 64)), qw, kw, cos, sin, pos, keys, values),     # partial head
        (qkv, qw, kw, Fake((639, 128)), Fake((639, 128)), pos, keys, values),  # table capacity
        (qkv, qw, kw, cos, sin, pos, Fake((1, 8, 640, 128)), Fake((1, 8, 640, 128))),  # batch
        (qkv, qw, kw, cos, sin, Fake((2,), torch.int64), keys, values),      # two positions
        (Fake((3, 24 * 64)), Fake((64,)), Fake((64,)), Fake((640, 64)), Fake((640, 64)), pos,
         Fake((3, 4, 640, 64)), Fake((3, 4, 640, 64))),                      # head width 64
    ]
    for args in bad:
        with pytest.raises(ValueError):
            decode_fused.qkv_norm_rope_cache(args[0], args[1], args[2], 0.0, 0.0, *args[3:])


# ------------------------------------------------------------- prefill_qkv

@pytest.mark.parametrize("b,t,c,nq,nk", [(4, 2048, 2080, 32, 8), (1, 3, 8, 4, 2), (2, 5, 9, 12, 4)])
def test_prefill_qkv_marshalling(b, t, c, nq, nk):
    qkv = Fake((b * t, (nq + 2 * nk) * 128))
    keys, values = Fake((b, nk, c, 128)), Fake((b, nk, c, 128))
    with recorded() as calls:
        q = prefill.prefill_qkv(qkv, Fake((128,)), Fake((128,)), 1e-6, 3e-6, Fake((c, 128)),
                                Fake((c, 128)), keys, values, t)
    assert tuple(q.shape) == (b, t, nq, 128)
    (name, *a), = calls
    assert name == "qf_prefill_qkv"
    assert a[:5] == [qkv.data_ptr(), b, t, nq, nk] and (a[7], a[8]) == (1e-6, 3e-6)
    assert a[11:15] == [c, q.data_ptr(), keys.data_ptr(), values.data_ptr()]


def test_prefill_qkv_rejects_bad_dimensions():
    args = (Fake((128,)), Fake((128,)), 1e-6, 1e-6, Fake((8, 128)), Fake((8, 128)))
    with pytest.raises(ValueError):  # rows disagree with B*T (tests/test_prefill.py:313-315)
        prefill.prefill_qkv(Fake((6, 6144)), *args, Fake((1, 8, 8, 128)), Fake((1, 8, 8, 128)), 3)
    with pytest.raises(ValueError):  # longer than the cache
        prefill.prefill_qkv(Fake((9, 6144)), *args, Fake((1, 8, 8, 128)), Fake((1, 8, 8, 128)), 9)
    with pytest.raises(ValueError):  # nq not a multiple of nk
        prefill.prefill_qkv(Fake((3, 13 * 128)), *args, Fake((1, 4, 8, 128)), Fake((1, 4, 8, 128)), 3)


# ---------------------------------------------------------------- embedding

def test_embedding_validation_and_shape():
    table = Fake((151936, 2560))
    with pytest.raises(ValueError):
        embedding.embedding(Fake((8,), torch.int32), table)
    with pytest.raises(ValueError):
        embedding.embedding(Fake((8,), torch.int64), Fake((10, 8), torch.float32))
    with recorded() as calls:
        ids = Fake((4, 2048), torch.int64)
        out = embedding.embedding(ids, table)
    assert tuple(out.shape) == (4, 2048, 2560)
    (name, *a), = calls
    assert a[:5] == [ids.data_ptr(), 8192, table.data_ptr(), 151936, 2560]


def test_fused_embedding_shares_the_weight_parameter():
    ref = torch.nn.Embedding(127, 64)
    fused = embedding.FusedEmbedding(ref)
    assert fused.weight is ref.weight
    with pytest.raises(ValueError):
        embedding.FusedEmbedding(torch.nn.Embedding(10, 8, max_norm=1.0))


def test_skinny_supports_is_the_reference_static_rule():
    """engine/kernels/skinny_gemm.py:75-83; the reference test's cases
    (tests/test_skinny_gemm.py:183-204) plus the 16-byte start alignment."""
    from starter_amd.kernels import skinny_gemm as sk
    x, w = Fake((4, 2560)), Fake((6144, 2560))
    assert sk.supports(x, w)
    assert sk.supports(Fake((sk.MAX_ROWS, 2560)), w)
    assert sk.supports(x, Fake((19456, 2560)), pairs=True)
    for bad_x, bad_w, pairs in (
        (Fake((sk.MAX_ROWS + 1, 2560)), w, False),
        (Fake((0, 2560)), w, False),
        (Fake((4, 2560), cuda=False), Fake((6144, 2560), cuda=False), False),
        (Fake((4, 2560), dtype=torch.float16), w, False),
        (Fake((4, 2560), strides=(1, 4)), w, False),
        (x, Fake((6144, 2560), strides=(1, 6144)), False),
        (Fake((4, 2570)), Fake((6144, 2570)), False),        # K not a multiple of 64
        (x, Fake((6144 + 8, 2560)), False),                  # N not a multiple of 32
        (x, Fake((3 * sk.BN, 2560)), True),                  # pairs need 2*BN
        (Fake((4, 2560)), Fake((6144, 2561)), False),        # K mismatch
        (Fake((2, 4, 2560)), w, False),
        (Fake((4, 2560), ptr=0x100008), w, False),           # misaligned start
    ):
        assert not sk.supports(bad_x, bad_w, pairs=pairs)
    with pytest.raises(ValueError):
        sk._dims(Fake((4, 2560), cuda=False), Fake((6144, 2560), cuda=False))
    with pytest.raises(ValueError):
        sk.linear_partials(Fake((65, 256)), Fake((64, 256)))
    with pytest.raises(ValueError):
        sk.linear_silu_mul(Fake((4, 256)), Fake((96, 256)))


def test_skinny_split_plan():
    """The library's plan.  Up to 16 rows: a power of two dividing K/64 that
    leaves every wave a chunk, fewer as rows grow (the partials cost rows *
    splits).  Beyond 16 rows: K ranges of at most eight chunks."""
    from starter_amd.kernels import skinny_gemm as sk
    qwen = {"qkv": (6144, 2560), "o": (2560, 4096), "down": (2560, 9728)}
    for n, k in qwen.values():
        prev = None
        for rows in (1, 4, 16):
            s = sk.split_count(n, k, rows)
            assert s >= 1 and s & (s - 1) == 0 and (k // 64) % s == 0 and k // 64 // s >= 4
            assert prev is None or s <= prev
            prev = s
        for rows in (17, 32, 48, 64):
            s = sk.split_count(n, k, rows)
            chunks = k // 64
            assert chunks % s == 0 and chunks // s <= 8
            assert not any(chunks % t == 0 and chunks // t <= 8 for t in range(1, s))  # the fewest
    assert sk.split_count(6144, 2560, 1) == 8 and sk.split_count(6144, 2560, 16) == 4
    assert sk.split_count(2560, 4096, 1) == 8 and sk.split_count(2560, 9728, 16) == 8
    assert [sk.split_count(n, k, 64) for n, k in qwen.values()] == [5, 8, 19]
    assert sk.split_count(6144, 2560, 32) == 5 and sk.split_count(2560, 4096, 48) == 8
    assert sk.split_count(1024, 64, 1) == 1      # one chunk: no split possible
    assert sk.split_count(1024, 64, 64) == 1
    with pytest.raises(ValueError):
        sk.split_count(6144, 2560, 65)
    with pytest.raises(ValueError):
        sk.split_count(6144 + 16, 2560, 1)


def test_skinny_marshalling():
    from starter_amd.kernels import skinny_gemm as sk
    with recorded() as calls:
        p = sk.linear_partials(Fake((5, 2560)), Fake((6144, 2560)))
        h = sk.linear_silu_mul(Fake((5, 2560)), Fake((19456, 2560)))
    assert tuple(p.shape) == (sk.split_count(6144, 2560, 5), 5, 6144) and p.dtype == torch.float32
    assert tuple(h.shape) == (5, 9728) and h.dtype == BF16
    name, _, m, k, _, n, splits = calls[0][:7]
    assert (name, m, k, n, splits) == ("qf_linear_partials", 5, 2560, 6144, p.shape[0])
    name, _, m, k, _, n = calls[1][:6]
    assert (name, m, k, n) == ("qf_linear_silu_mul", 5, 2560, 9728)


def test_skinny_merged_rule_and_marshalling():
    """o_proj over unmerged attention segments: Qwen3-4B's 32/8 heads at batch 1."""
    from starter_amd.kernels import skinny_gemm as sk
    f32 = torch.float32
    parts, stats, w = Fake((8, 9, 4, 128), f32), Fake((8, 9, 2, 4), f32), Fake((2560, 4096))
    assert sk.supports_merged(parts, stats, 1, w)
    with recorded() as calls:
        out = sk.linear_partials_merged(parts, stats, 1, w)
    splits = sk.split_count(2560, 4096, 1)
    assert tuple(out.shape) == (splits, 1, 2560) and out.dtype == f32
    name, pp, ps, segs, batch, hq, hk, pw, n, s, po = calls[0][:11]
    assert (name, segs, batch, hq, hk, n, s) == ("qf_linear_partials_merged", 9, 1, 32, 8, 2560, splits)
    assert (pp, ps, pw, po) == (parts.data_ptr(), stats.data_ptr(), w.data_ptr(), out.data_ptr())
    # batch 2 of the same heads: 16 virtual heads
    assert sk.supports_merged(Fake((16, 9, 4, 128), f32), Fake((16, 9, 2, 4), f32), 2, w)
    for bad in ((Fake((8, 1, 4, 128), f32), Fake((8, 1, 2, 4), f32), 1, w),     # one segment
                (parts, Fake((8, 9, 2, 2), f32), 1, w),                          # stats mismatch
                (parts, stats, 1, Fake((2560, 2048))),                           # k != Hq * 128
                (parts, stats, 3, w),                                            # 8 % 3
                (Fake((8, 9, 4, 128), BF16), stats, 1, w),
                (parts, stats, 1, Fake((2560, 4096), cuda=False))):
        assert not sk.supports_merged(*bad)
        with pytest.raises(ValueError):
            sk.linear_partials_merged(*bad)


def test_attention_partition_contract():
    """The reference test's grid (tests/test_small_query_attention.py:217-230)."""
    from starter_amd.kernels.small_query_attention import partition_keys
    for heads in (1, 8, 24, 128, 512, 4096):
        for capacity in (1, 63, 64, 65, 544, 2080, 8193, 262144):
            for units in (1, 80, 114, 132, 144, 256):
                splits, span = partition_keys(heads, capacity, units)
                assert 1 <= splits <= 32 and span % 64 == 0
                assert (splits - 1) * span < capacity <= splits * span
    for args in ((0, 1, 1), (1, 0, 1), (1, 1, 0)):
        with pytest.raises(ValueError):
            partition_keys(*args)


def test_aligned_attention_partition_contract():
    """The finer plan: the same coverage rules at 16/32/64-key granularity,
    the segment count partition_keys aims for (one per CU, <= 32, >= one
    64-key tile each), and the 64-key plan itself at align 64."""
    from starter_amd.kernels.small_query_attention import partition_keys, partition_keys_aligned
    for heads in (1, 8, 24, 32, 128, 512, 4096):
        for capacity in (1, 15, 16, 17, 63, 64, 65, 544, 545, 641, 2080, 2081, 8193, 262144):
            for units in (1, 80, 114, 256):
                aim = max(1, min(units // heads, -(-capacity // 64), 32))
                for align in (16, 32, 64):
                    splits, span = partition_keys_aligned(heads, capacity, units, align)
                    assert 1 <= splits <= aim and span % align == 0
                    assert (splits - 1) * span < capacity <= splits * span
                assert partition_keys_aligned(heads, capacity, units, 64) == partition_keys(heads, capacity, units)
    assert partition_keys_aligned(32, 2081, 256, 16) == (8, 272)
    for args in ((0, 1, 1, 16), (1, 0, 1, 16), (1, 1, 0, 16), (1, 1, 1, 8), (1, 1, 1, 128)):
        with pytest.raises(ValueError):
            partition_keys_aligned(*args)


def test_attention_context_validation_and_marshalling():
    from starter_amd.kernels import small_query_attention as sqa
    props = mock.Mock(multi_processor_count=256)
    fake = lambda shape, dtype, device: Fake(shape, dtype)  # noqa: E731
    with mock.patch.object(torch.cuda, "get_device_properties", return_value=props), \
            mock.patch.object(torch, "empty", side_effect=fake):
        for bad in ((1, 34, 2, 13, "cuda"), (1, 8, 3, 13, "cuda"), (0, 8, 2, 13, "cuda"),
                    (1, 8, 2, 13, "cpu")):
            with pytest.raises(ValueError):
                sqa.SmallQueryAttention(*bad)
        plan = sqa.SmallQueryAttention(2, 8, 2, 257, "cuda:0")
    assert (plan.groups, plan.virtual_heads) == (4, 4)
    assert (plan.splits, plan.span) == sqa.partition_keys(4, 257, 256)
    assert tuple(plan.partials.shape) == (4, plan.splits, 4, 128) and plan.partials.dtype == torch.float32
    assert tuple(plan.stats.shape) == (4, plan.splits, 2, 4)
    plan.partials.device = torch.device("cuda", 0)
    q, k = Fake((2, 8, 1, 128)), Fake((2, 2, 257, 128))
    used = Fake((4,), dtype=torch.int32)
    with recorded() as calls, torch.no_grad():
        out = plan.run(q, k, k, used, 0.25)
    assert tuple(out.shape) == (2, 1, 8, 128)
    name, *args = calls[0]
    assert name == "qf_decode_attention"
    assert args[4:11] == [2, 8, 2, 257, 0.25, plan.splits, plan.span]
    for bad_args in ((q, k, k, Fake((4,), dtype=torch.int64), 0.25),
                     (Fake((2, 8, 1, 128), dtype=torch.float32), k, k, used, 0.25),
                     (q, k, k, used, float("nan")),
                     (q, Fake((2, 2, 256, 128)), k, used, 0.25)):
        with pytest.raises(ValueError), torch.no_grad():
            plan.run(*bad_args)
    with pytest.raises(ValueError):  # autograd enabled
        plan.run(q, k, k, used, 0.25)
    # fused Q/K/V prologue: f32 partials or bf16 rows, gains, tables, device position
    parts = Fake((8, 2, (8 + 2 * 2) * 128), dtype=torch.float32)
    gain, table, pos = Fake((128,)), Fake((257, 128)), Fake((1,), dtype=torch.int64)
    with recorded() as calls, torch.no_grad():
        out = plan.run_qkv(parts, gain, gain, 1e-6, 2e-6, table, table, pos, k, k, used, 0.25)
        plan.run_qkv(Fake((2, 12 * 128)), gain, gain, 1e-6, 2e-6, table, table, pos, k, k, used, 0.5)
    assert tuple(out.shape) == (2, 1, 8, 128)
    name, *args = calls[0]
    assert name == "qf_decode_attention_qkv"
    assert args[1] == 8 and args[4:6] == [1e-6, 2e-6] and args[8] == pos.data_ptr()
    assert args[12:19] == [2, 8, 2, 257, 0.25, plan.splits, plan.span]
    assert calls[1][2] == 0  # bf16 rows: no partials
    good = [parts, gain, gain, 1e-6, 2e-6, table, table, pos, k, k, used, 0.25]
    for index, bad in ((0, Fake((8, 2, 11 * 128), dtype=torch.float32)),   # wrong packed width
                       (0, Fake((2, 12 * 128), dtype=torch.float16)),
                       (5, Fake((256, 128))),                                # table != capacity
                       (7, Fake((1,), dtype=torch.int32)),
                       (8, Fake((2, 2, 256, 128))),
                       (11, float("inf"))):
        with pytest.raises(ValueError), torch.no_grad():
            plan.run_qkv(*good[:index], bad, *good[index + 1:])
    # unmerged: same launch with no output (the segments stay in the scratch)
    with recorded() as calls, torch.no_grad():
        plan.run_qkv(*good)
        assert plan.run_qkv_unmerged(*good) is None
    assert calls[1][0] == "qf_decode_attention_qkv" and calls[1][-2] is None
    assert calls[1][:-2] == calls[0][:-2] and plan.splits > 1
    with mock.patch.object(torch.cuda, "get_device_properties", return_value=props), \
            mock.patch.object(torch, "empty", side_effect=fake):
        single = sqa.SmallQueryAttention(2, 8, 2, 64, "cuda:0")
    assert single.splits == 1
    with pytest.raises(ValueError), torch.no_grad():
        single.run_qkv_unmerged(*good)


def test_lm_head_rule_and_marshalling():
    from starter_amd.kernels import lm_head
    x, w = Fake((4, 2560)), Fake((151936, 2560))
    assert lm_head.supports(x, w)
    for bad_x, bad_w in ((Fake((65, 2560)), w), (x, Fake((151930, 2560))), (Fake((4, 2570)), Fake((16, 2570))),
                         (Fake((4, 2560), cuda=False), Fake((16, 2560), cuda=False))):
        assert not lm_head.supports(bad_x, bad_w)
    with pytest.raises(ValueError):
        lm_head.lm_head_argmax(Fake((4, 2560), dtype=torch.float32), w)
    with recorded() as calls:
        tokens, logits = lm_head.lm_head_argmax(x, w, logits=True)
    assert tuple(tokens.shape) == (4,) and tokens.dtype == torch.int64
    assert tuple(logits.shape) == (4, 151936)
    name, _, rows, k, _, vocab = calls[0][:6]
    assert (name, rows, k, vocab) == ("qf_lm_head_argmax", 4, 2560, 151936)
