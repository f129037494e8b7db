"""Rotary cos/sin tables for every cache slot, built on gfx950 HIP.

The engine builds ``[C, 128]`` bf16 tables once per shape from the model's own
rotary module (engine/decode.py:52-59, ``Qwen3RotaryEmbedding.forward``):
``ang = inv_freq (x) float(pos)`` in f32, ``cos/sin(cat(ang, ang))`` cast to
bf16.  ``rope_tables`` computes the same tables on the device from the
model's ``inv_freq`` buffer.
"""

from __future__ import annotations

import torch

from . import _lib


def default_inv_freq(theta: float, dim: int) -> torch.Tensor:
    """Qwen3 default RoPE inverse frequencies ``1 / theta**(arange(0, dim, 2) / dim)``
    in f32, evaluated the way the model's rotary module initialises its buffer
    (transformers ``Qwen3RotaryEmbedding.compute_default_rope_parameters``)."""
    exponent = torch.arange(0, dim, 2, dtype=torch.int64).float() / dim
    return 1.0 / (theta ** exponent)


def rope_tables(inv_freq: torch.Tensor, capacity: int | None = None, *,
                positions: torch.Tensor | None = None, start: int = 0,
                device: torch.device | str | None = None):
    """(cos, sin), each a contiguous bf16 ``[n, 2 * len(inv_freq)]`` tensor.

    Rows are slots ``start .. start + capacity - 1``, or the int64 device
    tensor ``positions`` (one row per entry) when given.
    """
    if positions is not None:
        if positions.dtype != torch.int64 or positions.ndim != 1 or not positions.is_cuda:
            raise ValueError("positions must be a 1-D int64 CUDA tensor")
        device = positions.device
        n = positions.numel()
        positions = positions.contiguous()
    else:
        if capacity is None or capacity < 0:
            raise ValueError("give capacity or positions")
        n = int(capacity)
    device = torch.device(device if device is not None else inv_freq.device)
    if device.type != "cuda":
        raise ValueError("rotary tables are built on a CUDA device")
    if inv_freq.ndim != 1 or inv_freq.numel() < 1:
        raise ValueError("inv_freq must be a non-empty 1-D tensor")
    inv = inv_freq.to(device=device, dtype=torch.float32).contiguous()
    half = inv.numel()
    cos = torch.empty((n, 2 * half), dtype=torch.bfloat16, device=device)
    sin = torch.empty_like(cos)
    if n:
        _lib.call("qf_rope_table", inv.data_ptr(), half, _lib.ptr(positions), int(start), n,
                  cos.data_ptr(), sin.data_ptr(), _lib.stream(device))
    return cos, sin
