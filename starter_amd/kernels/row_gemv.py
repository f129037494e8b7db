"""Decode projections at one to four rows with the residual add and the
RMSNorm folded into them (gfx950 HIP, one workgroup per compute unit).

The reference decode step (engine/decode_step.py:40-59) ends every layer with
``linear_partials`` (split-K f32 partials of the down projection) and
``add_rms_norm`` (residual add + RMSNorm of the next layer's input), and
starts the next layer with the qkv projection of that normalised row.  At
decode batch 1-4 the add + norm launch costs microseconds of latency for a
few KB, so here the down projection runs over the whole K range in 256
workgroups and adds the residual in its epilogue (``linear_residual``), and
the next projection normalises its input in its prologue (``linear_normed``)
from the per-workgroup sums of squares the first one wrote.  The normalised
row equals ``add_rms_norm``'s bit for bit (exact f64 sums of squares, the
same rounding steps); the projections accumulate in f32 over the whole K
range in a fixed order.

``supports`` is the shape rule; every call launches one kernel on torch's
current stream and allocates its outputs fresh.  No fallback: without the
HIP library every call raises.
"""

from __future__ import annotations

import math

import torch

from . import _lib

#: Workgroups per launch, and sums of squares per row (QF_ROW_GROUPS).
GROUPS = 256
MAX_ROWS = 4


def _aligned(t) -> bool:
    return t.data_ptr() % 16 == 0


def supports(x, weight) -> bool:
    """x bf16 [1..4, K] and W bf16 [N, K] on one device, contiguous and
    16-byte aligned, with N = 256 c for a column count c the library serves."""
    if not (x.ndim == 2 and weight.ndim == 2 and x.shape[1] == weight.shape[1]
            and x.is_cuda and weight.device == x.device
            and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and x.is_contiguous() and weight.is_contiguous()
            and 1 <= x.shape[0] <= MAX_ROWS and _aligned(x) and _aligned(weight)):
        return False
    return bool(_lib.lib().qf_row_supported(x.shape[0], x.shape[1], weight.shape[0]))


def supports_shape(rows: int, k: int, n: int) -> bool:
    """The shape rule alone: x [rows, k] @ W[n, k].T (no tensors needed)."""
    return 1 <= rows <= MAX_ROWS and bool(_lib.lib().qf_row_supported(rows, k, n))


def _check(x, weight):
    if not supports(x, weight):
        raise ValueError("expected contiguous BF16 CUDA X[1..4, K] and W[256c, K] "
                         "(c in 2, 4, 8, 10, 16, 24, 32)")
    return x.shape[0], weight.shape[0], x.shape[1]


def linear_rows(x, weight):
    """bf16(x @ weight.T), f32 accumulation over the whole K range."""
    rows, n, k = _check(x, weight)
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=x.device)
    _lib.call("qf_linear_rows", x.data_ptr(), rows, k, weight.data_ptr(), n, out.data_ptr(),
              _lib.stream(x.device))
    return out


def linear_residual(x, weight, residual):
    """(total, sq): total = bf16(residual + bf16(x @ weight.T)) [rows, N] and
    sq f64 [rows, 256], sq[r, g] = sum of total[r, j]^2 over workgroup g's
    columns j (N / 256 consecutive columns each)."""
    rows, n, k = _check(x, weight)
    if (residual.shape != (rows, n) or residual.dtype != torch.bfloat16
            or residual.device != x.device or not residual.is_contiguous()):
        raise ValueError("residual must be a contiguous BF16 [rows, N] tensor on x's device")
    total = torch.empty_like(residual)
    sq = torch.empty((rows, GROUPS), dtype=torch.float64, device=x.device)
    _lib.call("qf_linear_residual", x.data_ptr(), rows, k, weight.data_ptr(), n,
              residual.data_ptr(), total.data_ptr(), sq.data_ptr(), _lib.stream(x.device))
    return total, sq


def linear_normed(total, sq, gain, eps, weight):
    """bf16(RMSNorm(total) @ weight.T), the norm's inverse RMS taken from
    ``sq`` (as ``linear_residual`` wrote it for ``total``) and its rounding
    steps those of ``add_rms_norm``: bf16(bf16(total * inv) * gain)."""
    rows, n, k = _check(total, weight)
    if (sq.shape != (rows, GROUPS) or sq.dtype != torch.float64 or sq.device != total.device
            or not sq.is_contiguous()):
        raise ValueError("sq must be a contiguous float64 [rows, 256] tensor on total's device")
    if (gain.shape != (k,) or gain.dtype != torch.bfloat16 or gain.device != total.device
            or not gain.is_contiguous() or not _aligned(gain)):
        raise ValueError("gain must be a contiguous BF16 [K] tensor on total's device")
    if not (math.isfinite(eps) and eps >= 0):
        raise ValueError("eps must be finite and non-negative")
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=total.device)
    _lib.call("qf_linear_normed", total.data_ptr(), sq.data_ptr(), gain.data_ptr(), float(eps),
              rows, k, weight.data_ptr(), n, out.data_ptr(), _lib.stream(total.device))
    return out
