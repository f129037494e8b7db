"""Decode fusions that keep Qwen3's bf16 cast boundaries, on gfx950 HIP kernels.

Drop-in for ``engine/kernels/decode_fused.py`` (jadenpxrk/starter): the three
wrappers ``add_rms_norm``, ``silu_mul`` and ``qkv_norm_rope_cache`` keep their
names, signatures, validation (``ValueError`` before any launch), fresh output
allocation and the single in-place effect (the K/V cache slot).  They launch
on torch's current stream and never synchronise, so they are capturable into
a HIP graph.
"""

from __future__ import annotations

import torch

from . import _lib

#: Largest row width (as next power of two) the reference accepts
#: (engine/kernels/decode_fused.py:16); kept for identical errors.
MAX_BLOCK = 8192
HEAD = 128


def _next_power_of_2(n: int) -> int:
    return 1 << (n - 1).bit_length() if n > 0 else 1


def _rows(x):
    """(rows, cols) of ``x``, which must be a dense 2-D bf16 tensor on a GPU;
    anything else raises ValueError (engine/kernels/decode_fused.py:121-124)."""
    if x.ndim != 2 or not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("expected a contiguous 2-D BF16 CUDA tensor")
    return x.shape


def _splits(branch, shape, device):
    """How the kernel reads ``branch``: 0 when it is a bf16 matrix shaped like
    the residual, or the split count S when it is a dense f32 stack of S
    split-K partial products ``[S, rows, cols]``; any other operand raises
    ValueError (engine/kernels/decode_fused.py:127-137)."""
    if branch.ndim == 3 and branch.dtype == torch.float32:
        if (tuple(branch.shape[1:]) != tuple(shape) or branch.shape[0] < 1
                or branch.device != device or not branch.is_contiguous()):
            raise ValueError("split-K partials must be contiguous FP32 [splits, rows, cols]")
        return branch.shape[0]
    if tuple(branch.shape) != tuple(shape) or branch.device != device:
        raise ValueError("operand shape or device disagrees")
    _rows(branch)
    return 0


def add_rms_norm(residual, branch, weight, eps):
    """One launch for the two steps between sublayers: ``total`` = bf16 sum of
    the residual stream and the sublayer's output ``branch``, and ``normed``
    = RMSNorm of ``total`` with gain ``weight``; both are new bf16 tensors
    shaped like ``residual``, which is left as it was.

    A bf16 ``branch`` is added as is.  An f32 ``branch`` holds a projection's
    S split-K partials: the kernel sums them from split 0 upwards in f32 and
    rounds that sum to bf16 once before the add
    (engine/kernels/decode_fused.py:140-158 is the function this replaces).
    """
    n_rows, n_cols = _rows(residual)
    if tuple(weight.shape) != (n_cols,):
        raise ValueError("residual and gain shapes disagree")
    if weight.dtype != torch.bfloat16 or weight.device != residual.device:
        raise ValueError("gain must be BF16 on the residual's device")
    splits = _splits(branch, residual.shape, residual.device)
    if _next_power_of_2(n_cols) > MAX_BLOCK:
        raise ValueError(f"a row must fit in one block; {n_cols} columns does not")
    total, normed = torch.empty_like(residual), torch.empty_like(residual)
    if n_rows:
        weight = weight.contiguous()
        _lib.call("qf_add_rms_norm", residual.data_ptr(), branch.data_ptr(), splits,
                  weight.data_ptr(), n_rows, n_cols, float(eps), total.data_ptr(),
                  normed.data_ptr(), _lib.stream(residual.device))
    return total, normed


def silu_mul(gate_up, block=1024):
    """The MLP activation on a packed gate/up projection: row r of the
    ``[rows, 2N]`` input holds the N gate values, then the N up values; the
    new ``[rows, N]`` bf16 output holds bf16(bf16(SiLU(gate)) * up).

    ``block`` exists so calls written for engine/kernels/decode_fused.py:161
    still bind; the HIP kernel picks its own tiling and ignores it.
    """
    n_rows, width = _rows(gate_up)
    if width % 2:
        raise ValueError("packed gate/up width must be even")
    if int(block) < 1:
        raise ValueError("block must be positive")
    n_cols = width // 2
    out = torch.empty((n_rows, n_cols), dtype=gate_up.dtype, device=gate_up.device)
    if n_rows and n_cols:
        _lib.call("qf_silu_mul", gate_up.data_ptr(), n_rows, n_cols, out.data_ptr(),
                  _lib.stream(gate_up.device))
    return out


def qkv_norm_rope_cache(qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position,
                        key_cache, value_cache):
    """Decode step's Q/K head RMSNorm + RoPE with the K/V cache write.

    Input: one packed projection row per sequence, ``[q heads | k heads |
    v heads]`` of 128 each - bf16 ``[batch, width]``, or the f32 split-K
    partials ``[S, batch, width]`` that the kernel sums in order and rounds to
    bf16 first.  The rotary angle comes from row ``position`` of the
    ``[capacity, 128]`` cos/sin tables, with ``position`` an int64 ``(1,)``
    tensor read on the device.  The normalised, rotated key row and the copied
    value row go to slot ``position`` of ``key_cache`` / ``value_cache``
    (``[batch, Nkv, capacity, 128]``); no other slot changes.  Returns a new
    ``[batch, Nq, 1, 128]`` Q.  Contract of engine/kernels/decode_fused.py:
    172-210; unlike it, a position outside [0, capacity) writes nothing and
    the returned Q is all NaN.
    """
    if qkv.ndim == 3 and qkv.dtype == torch.float32:
        if not qkv.is_cuda or not qkv.is_contiguous() or qkv.shape[0] < 1:
            raise ValueError("split-K partials must be contiguous FP32 CUDA [splits, batch, width]")
        splits, (batch, width) = qkv.shape[0], qkv.shape[1:]
    else:
        splits, (batch, width) = 0, _rows(qkv)
    if (key_cache.ndim != 4 or key_cache.shape != value_cache.shape
            or key_cache.shape[0] != batch):
        raise ValueError("K/V caches must be [batch, Nkv, capacity, D]")
    _, kv_heads, capacity, head = key_cache.shape
    heads = width // head - 2 * kv_heads if head else 0
    if (head & (head - 1) or heads < 1 or width != (heads + 2 * kv_heads) * head
            or tuple(q_weight.shape) != (head,) or tuple(k_weight.shape) != (head,)
            or tuple(cos.shape) != (capacity, head) or sin.shape != cos.shape
            or tuple(position.shape) != (1,) or position.dtype != torch.int64):
        raise ValueError("unsupported packed Q/K/V, rotary table or position shape")
    if head != HEAD:
        raise ValueError(f"head width must be {HEAD}")
    tensors = (q_weight, k_weight, cos, sin, key_cache, value_cache)
    if (position.device != qkv.device or any(
            t.device != qkv.device or t.dtype != torch.bfloat16 or not t.is_contiguous()
            for t in tensors)):
        raise ValueError("Q/K/V fusion requires contiguous BF16 tensors on one CUDA device")
    q = torch.empty((batch, heads, 1, head), dtype=torch.bfloat16, device=qkv.device)
    if batch:
        _lib.call("qf_qkv_norm_rope_cache", qkv.data_ptr(), splits, batch, heads, kv_heads,
                  q_weight.data_ptr(), k_weight.data_ptr(), float(q_eps), float(k_eps),
                  cos.data_ptr(), sin.data_ptr(), position.data_ptr(), capacity, q.data_ptr(),
                  key_cache.data_ptr(), value_cache.data_ptr(), _lib.stream(qkv.device))
    return q
