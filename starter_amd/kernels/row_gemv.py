"""Decode projections at one to four rows with the residual add and the
RMSNorm folded into them (gfx950 HIP, one workgroup per compute unit).

The reference decode step (engine/decode_step.py:40-59) follows both the
attention's output projection and the down projection with ``add_rms_norm``
(residual add + RMSNorm of the next projection's input) over split-K f32
partials.  At decode batch 1-4 those add + norm launches cost microseconds
of latency for a few KB, so here a projection runs over the whole K range
in 256 workgroups and adds the residual in its epilogue
(``linear_residual``; ``linear_residual_merged`` for o_proj, merging the
attention's key segments in its prologue), and the next projection
normalises its input in its prologue (``linear_normed``;
``linear_silu_mul_normed`` for gate/up, with the SiLU * up epilogue) from
the per-workgroup sums of squares the first one wrote.  The normalised row
equals ``add_rms_norm``'s bit for bit (exact f64 sums of squares, the same
rounding steps) and the merged row the attention merge's; the projections
accumulate in f32 over the whole K range in a fixed order.

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


def supports_silu_shape(rows: int, k: int, n: int) -> bool:
    """x [rows, k] against a packed gate/up weight [2n, k]."""
    return 1 <= rows <= MAX_ROWS and bool(_lib.lib().qf_row_silu_supported(rows, k, n))


def supports_merged_shape(rows: int, segments: int, q_heads: int, kv_heads: int, n: int) -> bool:
    """o_proj [n, q_heads * 128] of the attention's ``segments`` key segments."""
    return bool(_lib.lib().qf_row_merged_supported(rows, segments, q_heads, kv_heads, n))


def linear_silu_mul_normed(total, sq, gain, eps, gate_up):
    """bf16(silu(g) * u) for the packed ``gate_up`` [2N, K] projections of
    RMSNorm(total) (the norm as ``linear_normed`` applies it); returns [rows, N]."""
    rows, k = total.shape if total.ndim == 2 else (0, 0)
    n = gate_up.shape[0] // 2 if gate_up.ndim == 2 else 0
    if not (total.ndim == 2 and gate_up.ndim == 2 and gate_up.shape[1] == k
            and total.is_cuda and gate_up.device == total.device
            and total.dtype == torch.bfloat16 and gate_up.dtype == torch.bfloat16
            and total.is_contiguous() and gate_up.is_contiguous()
            and _aligned(total) and _aligned(gate_up) and gate_up.shape[0] % 2 == 0
            and supports_silu_shape(rows, k, n)):
        raise ValueError("expected contiguous BF16 CUDA total[1..4, K] and gate_up[2N, K] "
                         "with 2N = 256c (c in 4, 8, 16, 32, 76)")
    if (sq.shape != (rows, GROUPS) or sq.dtype != torch.float64 or sq.device != total.device
            or not sq.is_contiguous()):
        raise ValueError("sq must be a contiguous float64 [rows, 256] tensor on total's device")
    if (gain.shape != (k,) or gain.dtype != torch.bfloat16 or gain.device != total.device
            or not gain.is_contiguous() or not _aligned(gain)):
        raise ValueError("gain must be a contiguous BF16 [K] tensor on total's device")
    if not (math.isfinite(eps) and eps >= 0):
        raise ValueError("eps must be finite and non-negative")
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=total.device)
    _lib.call("qf_linear_silu_mul_normed", total.data_ptr(), sq.data_ptr(), gain.data_ptr(),
              float(eps), rows, k, gate_up.data_ptr(), n, out.data_ptr(), _lib.stream(total.device))
    return out


def linear_residual_merged(partials, stats, batch, weight, residual):
    """``linear_residual`` of the attention output merged from its key
    segments (``partials`` [B*Hkv, S, G, 128] and ``stats`` [B*Hkv, S, 2, G],
    as ``SmallQueryAttention.run_qkv_unmerged`` leaves them)."""
    ok = (partials.ndim == 4 and stats.ndim == 4 and partials.dtype == torch.float32
          and stats.dtype == torch.float32 and partials.is_cuda and partials.is_contiguous()
          and stats.is_contiguous() and stats.device == partials.device
          and weight.ndim == 2 and weight.dtype == torch.bfloat16 and weight.is_contiguous()
          and weight.device == partials.device and _aligned(weight) and batch >= 1
          and partials.shape[0] % batch == 0 and partials.shape[3] == 128)
    if ok:
        kv_heads = partials.shape[0] // batch
        segments, groups = partials.shape[1], partials.shape[2]
        q_heads = kv_heads * groups
        n = weight.shape[0]
        ok = (tuple(stats.shape) == (batch * kv_heads, segments, 2, groups)
              and weight.shape[1] == q_heads * 128
              and supports_merged_shape(batch, segments, q_heads, kv_heads, n))
    if not ok:
        raise ValueError("expected contiguous FP32 attention segments [B*Hkv, S, G, 128] / "
                         "[B*Hkv, S, 2, G] and a BF16 CUDA weight [256c, Hq*128]")
    if (residual.shape != (batch, n) or residual.dtype != torch.bfloat16
            or residual.device != weight.device or not residual.is_contiguous()):
        raise ValueError("residual must be a contiguous BF16 [batch, N] tensor on the weight's device")
    total = torch.empty_like(residual)
    sq = torch.empty((batch, GROUPS), dtype=torch.float64, device=weight.device)
    _lib.call("qf_linear_residual_merged", partials.data_ptr(), stats.data_ptr(), segments, batch,
              q_heads, kv_heads, weight.data_ptr(), n, residual.data_ptr(), total.data_ptr(),
              sq.data_ptr(), _lib.stream(weight.device))
    return total, sq
