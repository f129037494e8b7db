"""Grouped-query decode attention on gfx950 (split-KV with an f32 merge).

Drop-in for ``engine/kernels/small_query_attention.py`` (jadenpxrk/starter),
which ``engine/flash_decode.py:48-52`` imports for CUDA GQA with at most 16
query heads per KV head: ``partition_keys`` and ``SmallQueryAttention`` keep
their names, signatures, ``ValueError`` rules, scratch ownership (one context
per instance, calls serialised on one stream) and fresh output allocation.

One query token per sequence attends the first ``used[b * Hkv + h]`` keys of
its KV head in the head-major cache; slots beyond that are never read.
Softmax statistics and the value accumulation stay f32; the probabilities
that multiply V are rounded to bf16 and only the merged output is rounded to
bf16 (engine/kernels/small_query_attention.py:1-9).  The work launches on
torch's current stream with no host sync, so a captured decode step replays
it with fresh ``used`` lengths.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

QUERY_TILE = 16   # most query heads per KV head (engine/kernels/small_query_attention.py:18)
KEY_TILE = 64     # segment granularity in keys
MAX_SPLITS = 32
HEAD = 128


def partition_keys(virtual_heads, capacity, multiprocessors):
    """(splits, span): key segments of whole KEY_TILE tiles covering capacity,
    at most one workgroup per compute unit, at most MAX_SPLITS.  Metadata only;
    the valid length is read on the device.  Same contract as
    engine/kernels/small_query_attention.py:24-38."""
    if min(virtual_heads, capacity, multiprocessors) < 1:
        raise ValueError("positive head count, capacity and SM count required")
    splits, span = ctypes.c_int32(), ctypes.c_int64()
    _lib.call("qf_attention_partition", int(virtual_heads), int(capacity), int(multiprocessors),
              ctypes.byref(splits), ctypes.byref(span))
    return splits.value, span.value


def partition_keys_aligned(virtual_heads, capacity, multiprocessors, align):
    """partition_keys' segment count with the segment lengths balanced to
    ``align`` (16, 32 or 64) keys instead of whole KEY_TILE tiles: the decode
    attention accepts any multiple of 16, and at 4 sequences x 2081 keys 8
    segments of 272 keys (one workgroup per CU) take 10.6 us against 11.3 for
    partition_keys' 7 x 320.  Not part of the reference's contract, which
    fixes KEY_TILE multiples."""
    if min(virtual_heads, capacity, multiprocessors) < 1 or align not in (16, 32, 64):
        raise ValueError("positive head count, capacity and SM count and an align of 16, 32 or 64 required")
    splits, span = ctypes.c_int32(), ctypes.c_int64()
    _lib.call("qf_attention_partition_aligned", int(virtual_heads), int(capacity), int(multiprocessors),
              int(align), ctypes.byref(splits), ctypes.byref(span))
    return splits.value, span.value


class SmallQueryAttention:
    """Decode attention for one shape, fixed at construction (batch, query and
    key/value heads, cache capacity): each call attends B one-token queries
    over the first ``used`` keys of their K/V cache rows and writes a new bf16
    ``[B, 1, Hq, 128]`` result; the caches are only read.

    ``used`` is a dense int32 vector of B*Hkv key counts, each in
    [0, capacity], one per (sequence, key/value head).  The instance owns
    the f32 buffers its key segments merge through, so two calls in flight
    at once (other streams or threads) would overwrite each other's
    partials: issue them on one stream
    (engine/kernels/small_query_attention.py:113-158 is the class this
    replaces).  ``key_align`` (not in the reference) picks the segment
    granularity: KEY_TILE keeps partition_keys' plan, 16 or 32 balance the
    same number of segments more finely (partition_keys_aligned).
    """

    def __init__(self, batch, query_heads, kv_heads, capacity, device, key_align=KEY_TILE):
        device = torch.device(device)
        if (device.type != "cuda" or min(batch, query_heads, kv_heads, capacity) < 1
                or query_heads % kv_heads or not 1 <= query_heads // kv_heads <= QUERY_TILE):
            raise ValueError("unsupported small-query attention metadata")
        self.batch, self.hq, self.hk, self.capacity = batch, query_heads, kv_heads, capacity
        self.groups = query_heads // kv_heads
        self.virtual_heads = batch * kv_heads
        units = torch.cuda.get_device_properties(device).multi_processor_count
        if key_align == KEY_TILE:
            self.splits, self.span = partition_keys(self.virtual_heads, capacity, units)
        else:
            self.splits, self.span = partition_keys_aligned(self.virtual_heads, capacity, units, key_align)
        self.partials = torch.empty((self.virtual_heads, self.splits, self.groups, HEAD),
                                    dtype=torch.float32, device=device)
        self.stats = torch.empty((self.virtual_heads, self.splits, 2, self.groups),
                                 dtype=torch.float32, device=device)

    def run(self, query, key, value, used, scale):
        device = self.partials.device
        if (torch.is_grad_enabled() or not math.isfinite(scale)
                or query.shape != (self.batch, self.hq, 1, HEAD)
                or key.shape != (self.batch, self.hk, self.capacity, HEAD)
                or value.shape != key.shape
                or used.shape != (self.virtual_heads,) or used.dtype != torch.int32
                or used.device != device or not used.is_contiguous()
                or any(t.dtype != torch.bfloat16 or t.device != device or not t.is_contiguous()
                       for t in (query, key, value))):
            raise ValueError("expected fixed-shape contiguous BF16 CUDA Q/K/V and int32 lengths")
        out = torch.empty((self.batch, 1, self.hq, HEAD), dtype=torch.bfloat16, device=device)
        _lib.call("qf_decode_attention", query.data_ptr(), key.data_ptr(), value.data_ptr(),
                  used.data_ptr(), self.batch, self.hq, self.hk, self.capacity, float(scale),
                  self.splits, self.span, self.partials.data_ptr(), self.stats.data_ptr(),
                  out.data_ptr(), _lib.stream(device))
        return out

    def run_qkv(self, qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position,
                key_cache, value_cache, used, scale):
        """``qkv_norm_rope_cache`` followed by ``run`` on its Q, in the attention
        launches: the call pair engine/decode_step.py:43-47 makes, with the
        same arguments and the same results bit for bit (the new K/V row lands
        in slot ``position`` of the caches, Q never goes to memory).  ``qkv``
        is BF16 [B, (Hq + 2 Hkv) * 128] or FP32 split-K partials [S, B, ...]."""
        return self._qkv(qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position, key_cache,
                         value_cache, used, scale, merge=True)

    def run_qkv_unmerged(self, qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position,
                         key_cache, value_cache, used, scale):
        """``run_qkv`` without the segment merge: the per-segment partials and
        statistics stay in ``self.partials`` / ``self.stats`` (valid until the
        next call on this instance) for ``skinny_gemm.linear_partials_merged``,
        which merges them inside the o_proj projection.  Needs ``splits > 1``;
        returns None."""
        if self.splits < 2:
            raise ValueError("unmerged attention needs more than one key segment")
        self._qkv(qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position, key_cache,
                  value_cache, used, scale, merge=False)

    def _qkv(self, qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position, key_cache,
             value_cache, used, scale, merge):
        device = self.partials.device
        width = (self.hq + 2 * self.hk) * HEAD
        if qkv.dtype == torch.float32 and qkv.ndim == 3:
            qkv_splits = qkv.shape[0]
            ok = qkv_splits >= 1 and tuple(qkv.shape[1:]) == (self.batch, width)
        else:
            qkv_splits = 0
            ok = qkv.dtype == torch.bfloat16 and tuple(qkv.shape) == (self.batch, width)
        bf16 = (q_weight, k_weight, cos, sin, key_cache, value_cache)
        if (torch.is_grad_enabled() or not ok or not qkv.is_contiguous() or qkv.device != device
                or not math.isfinite(scale)
                or tuple(q_weight.shape) != (HEAD,) or tuple(k_weight.shape) != (HEAD,)
                or tuple(cos.shape) != (self.capacity, HEAD) or sin.shape != cos.shape
                or tuple(position.shape) != (1,) or position.dtype != torch.int64
                or position.device != device
                or key_cache.shape != (self.batch, self.hk, self.capacity, HEAD)
                or value_cache.shape != key_cache.shape
                or used.shape != (self.virtual_heads,) or used.dtype != torch.int32
                or used.device != device or not used.is_contiguous()
                or any(t.dtype != torch.bfloat16 or t.device != device or not t.is_contiguous()
                       for t in bf16)):
            raise ValueError("expected packed BF16 Q/K/V (or FP32 partials), BF16 gains, rotary "
                             "tables and caches, an int64 position and int32 lengths on one device")
        out = (torch.empty((self.batch, 1, self.hq, HEAD), dtype=torch.bfloat16, device=device)
               if merge else None)
        _lib.call("qf_decode_attention_qkv", qkv.data_ptr(), qkv_splits, q_weight.data_ptr(),
                  k_weight.data_ptr(), float(q_eps), float(k_eps), cos.data_ptr(), sin.data_ptr(),
                  position.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
                  used.data_ptr(), self.batch, self.hq, self.hk, self.capacity, float(scale),
                  self.splits, self.span, self.partials.data_ptr(), self.stats.data_ptr(),
                  out.data_ptr() if merge else None, _lib.stream(device))
        return out
