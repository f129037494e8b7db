"""Decode-sized projections on the gfx950 matrix cores (split-K weight streams).

Drop-in for ``engine/kernels/skinny_gemm.py`` (jadenpxrk/starter), imported by
``engine/decode_step.py:19-30``: ``supports``, ``linear_partials`` and
``linear_silu_mul`` keep their names, signatures, ``ValueError`` rule and
fresh output allocation; ``split_count`` takes the row count as an optional
third argument because the split plan here depends on it.

* ``linear_partials(x, weight)``: FP32 split-K partial sums ``[S, M, N]`` of
  ``x @ weight.T``.  ``add_rms_norm`` and ``qkv_norm_rope_cache`` add the S
  partials in order and round once to BF16.
* ``linear_partials_merged(partials, stats, batch, weight)``: the same partials
  for x = the decode attention's output, merged from its unmerged key
  segments inside the projection (no merge launch, x never in memory).
* ``linear_silu_mul(x, gate_up_weight)``: ``bf16(silu(bf16(gate)) * bf16(up))``
  for a packed ``[2N, K]`` weight, with both projections and the SiLU epilogue
  in one launch.
* ``linear_partials_normed`` / ``linear_silu_mul_normed``: the same two at 1-4
  rows for x = RMSNorm of the residual stream, normalised by each workgroup
  from the per-workgroup sums of squares ``row_gemv.linear_residual`` writes
  (no add + norm launch before them); bit-identical to the plain calls on
  ``add_rms_norm``'s normalised row.

Both launch one HIP kernel on torch's current stream (no host sync, no device
value read), so the engine's graph capture of the decode step takes them
unchanged.  There is no fallback: without the HIP library every call raises.
"""

from __future__ import annotations

import math

import torch

from . import _lib

#: Shape rule of the reference (engine/kernels/skinny_gemm.py:20-22): at most
#: 64 rows of x, N a multiple of BN (2*BN for packed pairs), K of BK.
MAX_ROWS = 64
BN = 32
BK = 64


def _aligned(t) -> bool:
    data_ptr = getattr(t, "data_ptr", None)
    return data_ptr is None or data_ptr() % 16 == 0


def supports(x, weight, pairs=False):
    """Static shape/dtype/layout rule; identical for every call of one shape.

    Same rule as engine/kernels/skinny_gemm.py:75-83, plus the 16-byte start
    alignment the vector loads need (a fresh or contiguous-from-offset-0
    tensor always has it).
    """
    columns = 2 * BN if pairs else BN
    return (x.ndim == 2 and weight.ndim == 2 and x.shape[1] == weight.shape[1]
            and x.is_cuda and weight.device == x.device
            and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and x.is_contiguous() and weight.is_contiguous()
            and 1 <= x.shape[0] <= MAX_ROWS
            and weight.shape[0] % columns == 0 and x.shape[1] % BK == 0
            and _aligned(x) and _aligned(weight))


def split_count(n, k, rows=1):
    """K splits of ``linear_partials`` for x [rows, k] @ W[n, k].T.

    Each split covers an equal run of whole 64-wide k chunks, so the count
    divides k / 64: a power of two up to 16 rows; beyond, K ranges of about
    512 per workgroup (5, 8 and 19 splits on the Qwen3-4B shapes).  The plan
    lives in the library (qf_linear_splits) so C callers get the same one;
    compare engine/kernels/skinny_gemm.py:86-91, which ignores rows.
    """
    status = _lib.lib().qf_linear_splits(int(rows), int(k), int(n))
    if status < 1:
        raise ValueError(f"no split plan for rows={rows}, n={n}, k={k}")
    return status


def _dims(x, weight, pairs=False):
    if not supports(x, weight, pairs):
        raise ValueError("expected contiguous BF16 CUDA X[M<=64,K] and W[N,K] with tile-aligned N, K")
    return x.shape[0], weight.shape[0], x.shape[1]


def linear_partials(x, weight):
    """FP32 split-K partials [S, M, N] of x @ weight.T; inputs are read-only.

    Mirrors engine/kernels/skinny_gemm.py:100-109.
    """
    m, n, k = _dims(x, weight)
    splits = split_count(n, k, m)
    partials = torch.empty((splits, m, n), dtype=torch.float32, device=x.device)
    _lib.call("qf_linear_partials", x.data_ptr(), m, k, weight.data_ptr(), n, splits,
              partials.data_ptr(), _lib.stream(x.device))
    return partials


#: Most rows (sequences) ``linear_partials_merged`` takes.
MERGED_MAX_ROWS = 16


def _merged_dims(partials, stats, batch, weight):
    """(segments, q_heads, kv_heads, n, k, splits) or None when the merged
    projection does not apply to these operands."""
    if (partials.ndim != 4 or stats.ndim != 4 or weight.ndim != 2 or not 1 <= batch <= MERGED_MAX_ROWS
            or partials.dtype != torch.float32 or stats.dtype != torch.float32
            or weight.dtype != torch.bfloat16 or not weight.is_cuda
            or partials.device != weight.device or stats.device != weight.device
            or not (partials.is_contiguous() and stats.is_contiguous() and weight.is_contiguous())):
        return None
    vheads, segments, groups, width = partials.shape
    if (width != 128 or tuple(stats.shape) != (vheads, segments, 2, groups) or vheads % batch
            or not 2 <= segments <= 32 or not 1 <= groups <= 16):
        return None
    kv_heads = vheads // batch
    q_heads = kv_heads * groups
    n, k = weight.shape
    if k != q_heads * 128 or n % BN or not _aligned(weight):
        return None
    splits = split_count(n, k, batch)
    chunks = k // BK // splits
    if chunks % 2 or batch * (chunks * BK * 2 + 16) > 64 * 1024:
        return None
    return segments, q_heads, kv_heads, n, k, splits


def supports_merged(partials, stats, batch, weight):
    """Whether ``linear_partials_merged`` takes these operands (a static rule)."""
    return _merged_dims(partials, stats, batch, weight) is not None


def linear_partials_merged(partials, stats, batch, weight):
    """FP32 split-K partials [S, batch, N] of ``attended @ weight.T``, where
    ``attended`` [batch, Hq * 128] is the merge of the attention's unmerged
    key segments (``partials`` [B*Hkv, segments, G, 128] and ``stats``
    [B*Hkv, segments, 2, G], as ``SmallQueryAttention.run_qkv_unmerged``
    leaves them).  Bit-identical to ``linear_partials`` of the merged
    attention output; replaces the hand-off engine/decode_step.py:48-52."""
    dims = _merged_dims(partials, stats, batch, weight)
    if dims is None:
        raise ValueError("expected contiguous FP32 attention segments [V, S, G, 128] / [V, S, 2, G] "
                         "and a BF16 CUDA weight [N, Hq*128] the merged plan covers")
    segments, q_heads, kv_heads, n, k, splits = dims
    out = torch.empty((splits, batch, n), dtype=torch.float32, device=weight.device)
    _lib.call("qf_linear_partials_merged", partials.data_ptr(), stats.data_ptr(), segments, batch,
              q_heads, kv_heads, weight.data_ptr(), n, splits, out.data_ptr(),
              _lib.stream(weight.device))
    return out


#: Most rows the normalising projections take; sums of squares per row.
NORMED_MAX_ROWS = 4
SQ_GROUPS = 256


def _normed_dims(total, sq, gain, eps, weight, pairs):
    """(rows, k, n) of a normalising call, raising ValueError like the
    plain calls for shapes, dtypes and layouts they do not take."""
    if not supports(total, weight, pairs) or total.shape[0] > NORMED_MAX_ROWS:
        raise ValueError("expected contiguous BF16 CUDA total[1..4, K] and W[N, K] with "
                         "tile-aligned N, K")
    rows, k = total.shape
    if (sq.shape != (rows, SQ_GROUPS) or sq.dtype != torch.float64 or sq.device != total.device
            or not sq.is_contiguous()):
        raise ValueError("sq must be a contiguous float64 [rows, 256] tensor on total's device")
    if (gain.shape != (k,) or gain.dtype != torch.bfloat16 or gain.device != total.device
            or not gain.is_contiguous() or not _aligned(gain)):
        raise ValueError("gain must be a contiguous BF16 [K] tensor on total's device")
    if not (math.isfinite(eps) and eps >= 0):
        raise ValueError("eps must be finite and non-negative")
    n = weight.shape[0] // 2 if pairs else weight.shape[0]
    return rows, k, n


def supports_normed_shape(rows, k, n, pairs=False):
    """Shape rule of the normalising calls for total [rows, k] against W [n, k]
    (``pairs``: a packed gate/up weight of 2n rows): the plain rule at 1-4
    rows, and each workgroup's normalised slice (rows x K / splits, whole K
    for gate/up) at most 10,240 values (5 16-byte pieces per thread)."""
    if not (1 <= rows <= NORMED_MAX_ROWS and k > 0 and n > 0 and k % BK == 0 and n % BN == 0):
        return False
    per_split = k if pairs else k // split_count(n, k, rows)
    return rows * per_split <= 10240


def linear_partials_normed(total, sq, gain, eps, weight):
    """``linear_partials(RMSNorm(total), weight)`` with the norm applied inside
    the projection: x = bf16(bf16(total * inv) * gain), inv from ``sq`` (the
    f64 [rows, 256] sums of squares ``row_gemv.linear_residual`` wrote for
    ``total``).  Same split plan and bits as the plain call on that x."""
    rows, k, n = _normed_dims(total, sq, gain, eps, weight, False)
    splits = split_count(n, k, rows)
    if not supports_normed_shape(rows, k, n):
        raise ValueError("the normalised slice of this shape exceeds 10,240 values per workgroup")
    partials = torch.empty((splits, rows, n), dtype=torch.float32, device=total.device)
    _lib.call("qf_linear_partials_normed", total.data_ptr(), sq.data_ptr(), gain.data_ptr(),
              float(eps), rows, k, weight.data_ptr(), n, splits, partials.data_ptr(),
              _lib.stream(total.device))
    return partials


def linear_silu_mul_normed(total, sq, gain, eps, gate_up_weight):
    """``linear_silu_mul(RMSNorm(total), gate_up_weight)`` with the norm as in
    ``linear_partials_normed``; returns BF16 [rows, N]."""
    rows, k, n = _normed_dims(total, sq, gain, eps, gate_up_weight, True)
    if not supports_normed_shape(rows, k, n, pairs=True):
        raise ValueError("the normalised row of this shape exceeds 10,240 values per workgroup")
    out = torch.empty((rows, n), dtype=torch.bfloat16, device=total.device)
    _lib.call("qf_linear_silu_mul_normed_tiled", total.data_ptr(), sq.data_ptr(), gain.data_ptr(),
              float(eps), rows, k, gate_up_weight.data_ptr(), n, out.data_ptr(),
              _lib.stream(total.device))
    return out


def linear_silu_mul(x, gate_up_weight):
    """BF16 silu(x @ gate.T) * (x @ up.T) for a packed [2N, K] weight; returns [M, N].

    Mirrors engine/kernels/skinny_gemm.py:112-121.
    """
    m, width, k = _dims(x, gate_up_weight, pairs=True)
    n = width // 2
    out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    _lib.call("qf_linear_silu_mul", x.data_ptr(), m, k, gate_up_weight.data_ptr(), n,
              out.data_ptr(), _lib.stream(x.device))
    return out
