"""Packed prefill Q/K head norm, RoPE, and full-prefix static-cache writes (gfx950 HIP).

Drop-in for ``engine/kernels/prefill.py`` (jadenpxrk/starter): same
signature, validation and outputs.  Q is [B,T,Hq,128]; K/V keep the
[B,Hkv,C,128] cache storage and only slots [0, T) are written.  Inputs and
the angle tables are read-only.

``prefill_attention`` is the causal attention the reference prefill runs next
on those tensors with torch's flash kernel (engine/prefill.py:13-23), as one
HIP launch of this package.
"""

from __future__ import annotations

import math

import torch

from . import _lib

HEAD = 128


def prefill_qkv(qkv, qw, kw, qeps, keps, cos, sin, keys, values, length):
    """Prompt-wide Q/K head RMSNorm + RoPE with the K/V cache fill.

    ``qkv`` holds one packed ``[q heads | k heads | v heads]`` row per prompt
    token (bf16 ``[B * T, (Hq + 2 Hkv) * 128]``); token t of a sequence sits
    at position t, so its angles are row t of the ``[C, 128]`` cos/sin tables.
    Keys (normalised and rotated) and values (copied) fill slots [0, T) of the
    ``[B, Hkv, C, 128]`` caches and nothing else; the inputs are not written.
    Returns a new contiguous bf16 Q ``[B, T, Hq, 128]``.  Every tensor on one
    device.  Contract of engine/kernels/prefill.py:66-96.
    """
    if keys.ndim != 4 or values.shape != keys.shape:
        raise ValueError("K/V must have matching [B,Hkv,C,D] shapes")
    batch, nk, capacity, width = keys.shape
    if (batch < 1 or nk < 1 or width != HEAD or not 1 <= length <= capacity
            or qkv.ndim != 2 or qkv.shape[0] != batch * length):
        raise ValueError("unsupported full-prefill dimensions")
    nq = qkv.shape[1] // width - 2 * nk
    if (nq < 1 or nq % nk or qkv.shape[1] != (nq + 2 * nk) * width
            or tuple(qw.shape) != (width,) or kw.shape != qw.shape
            or tuple(cos.shape) != (capacity, width) or sin.shape != cos.shape):
        raise ValueError("packed QKV, gains, or rotary tables disagree")
    tensors = (qkv, qw, kw, cos, sin, keys, values)
    if (not qkv.is_cuda or any(t.device != qkv.device or t.dtype != torch.bfloat16
                              or not t.is_contiguous() for t in tensors)):
        raise ValueError("prefill requires contiguous BF16 tensors on one CUDA device")
    q = torch.empty((batch, length, nq, width), device=qkv.device, dtype=qkv.dtype)
    _lib.call("qf_prefill_qkv", qkv.data_ptr(), batch, int(length), nq, nk, qw.data_ptr(),
              kw.data_ptr(), float(qeps), float(keps), cos.data_ptr(), sin.data_ptr(), capacity,
              q.data_ptr(), keys.data_ptr(), values.data_ptr(), _lib.stream(qkv.device))
    return q


def prefill_attention(q, keys, values, length, scale):
    """Causal attention of the prompt over its own cache slots.

    ``q`` is the bf16 ``[B, T, Hq, 128]`` that ``prefill_qkv`` returns,
    ``keys`` / ``values`` the ``[B, Hkv, C, 128]`` caches it filled; position t
    attends slots 0..t (T = ``length``), query head h the KV head h // (Hq /
    Hkv), with weights softmax(q . k * scale).  Returns a new bf16
    ``[B, T, Hq, 128]``; nothing is written to the inputs.  The reference
    computes this with aten._flash_attention_forward(is_causal=True) on
    ``keys[:, :, :T]`` / ``values[:, :, :T]`` (engine/prefill.py:13-23).
    """
    if keys.ndim != 4 or values.shape != keys.shape or q.ndim != 4:
        raise ValueError("expected Q [B,T,Hq,D] and K/V caches [B,Hkv,C,D]")
    batch, nk, capacity, width = keys.shape
    if (width != HEAD or tuple(q.shape[:2]) != (batch, length) or q.shape[3] != HEAD
            or not 1 <= length <= capacity):
        raise ValueError("unsupported prefill attention dimensions")
    nq = q.shape[2]
    if nq < 1 or nq % nk or nq // nk not in (1, 2, 4, 8):
        raise ValueError("query heads must be 1, 2, 4 or 8 per KV head")
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    tensors = (q, keys, values)
    if (not q.is_cuda or any(t.device != q.device or t.dtype != torch.bfloat16
                             or not t.is_contiguous() for t in tensors)):
        raise ValueError("prefill attention requires contiguous BF16 tensors on one CUDA device")
    out = torch.empty_like(q)
    _lib.call("qf_prefill_attention", q.data_ptr(), keys.data_ptr(), values.data_ptr(), batch,
              int(length), nq, nk, capacity, float(scale), out.data_ptr(), _lib.stream(q.device))
    return out
