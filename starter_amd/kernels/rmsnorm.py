"""Fused RMSNorm with Qwen3's bf16 cast placement, on the gfx950 HIP kernel.

Drop-in for ``engine/kernels/rmsnorm.py`` (jadenpxrk/starter): same name,
signature, shape rule and ``ValueError`` conditions.  The cast sits before the
gain multiply (``self.weight * hidden_states.to(input_dtype)`` in
Qwen3RMSNorm): ``y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)``.
"""

from __future__ import annotations

import torch

from . import _lib

#: One row must fit in one block in the reference (engine/kernels/rmsnorm.py:9);
#: the same limit on the row width is kept so callers see the same errors.
MAX_BLOCK = 8192


def _next_power_of_2(n: int) -> int:
    return 1 << (n - 1).bit_length() if n > 0 else 1


def _row_walk(x: torch.Tensor):
    """Describe the rows of ``x``'s last dimension as a two-level walk
    ``(rows, inner, outer_stride, inner_stride, tensor)``, copying only when
    no such walk exists (the reference always copies strided inputs,
    engine/kernels/rmsnorm.py:46)."""
    cols = x.shape[-1]
    if cols > 1 and x.stride(-1) != 1:
        x = x.contiguous()
    dims = [(size, stride) for size, stride in zip(x.shape[:-1], x.stride()[:-1]) if size != 1]
    merged: list[tuple[int, int]] = []
    for size, stride in dims:
        if merged and merged[-1][1] == stride * size:
            merged[-1] = (merged[-1][0] * size, stride)
        else:
            merged.append((size, stride))
    if not merged:
        return 1, 1, 0, 0, x
    if len(merged) == 1:
        size, stride = merged[0]
        return size, size, 0, stride, x
    if len(merged) == 2:
        (s0, st0), (s1, st1) = merged
        return s0 * s1, s1, st0, st1, x
    x = x.contiguous()
    rows = x.numel() // cols
    return rows, rows, 0, cols, x


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Normalise every length-C row of ``x`` (C = ``weight.numel()``, its last
    dimension) by the root mean square of its f32 values, then apply the
    bf16 gain ``weight`` - the arithmetic and rounding of Qwen3RMSNorm.

    Both operands are bf16 on one GPU; ``x`` may be a strided view.  The
    result is a new contiguous tensor shaped like ``x``
    (engine/kernels/rmsnorm.py:39-62 is the function this replaces).
    """
    shape = x.shape
    if x.ndim == 0:
        raise ValueError("rms_norm needs at least one dimension")
    n_cols = shape[-1]
    if n_cols < 1 or _next_power_of_2(n_cols) > MAX_BLOCK:
        raise ValueError(f"a row must fit in one block; {n_cols} columns does not")
    if (not x.is_cuda or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16
            or weight.device != x.device or tuple(weight.shape) != (n_cols,)):
        raise ValueError("rms_norm requires BF16 x and [cols] BF16 weight on one CUDA device")
    out = torch.empty(shape, dtype=x.dtype, device=x.device)
    if x.numel() == 0:
        return out
    weight = weight.contiguous()
    rows, inner, outer_stride, inner_stride, src = _row_walk(x)
    _lib.call("qf_rms_norm", src.data_ptr(), rows, n_cols, inner, outer_stride, inner_stride,
              weight.data_ptr(), float(eps), out.data_ptr(), _lib.stream(x.device))
    return out
