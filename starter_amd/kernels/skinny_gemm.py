"""Decode-sized projections on the gfx950 matrix cores (split-K weight streams).

Drop-in for ``engine/kernels/skinny_gemm.py`` (jadenpxrk/starter), imported by
``engine/decode_step.py:19-30``: ``supports``, ``linear_partials`` and
``linear_silu_mul`` keep their names, signatures, ``ValueError`` rule and
fresh output allocation; ``split_count`` takes the row count as an optional
third argument because the split plan here depends on it.

* ``linear_partials(x, weight)``: FP32 split-K partial sums ``[S, M, N]`` of
  ``x @ weight.T``.  ``add_rms_norm`` and ``qkv_norm_rope_cache`` add the S
  partials in order and round once to BF16.
* ``linear_silu_mul(x, gate_up_weight)``: ``bf16(silu(bf16(gate)) * bf16(up))``
  for a packed ``[2N, K]`` weight, with both projections and the SiLU epilogue
  in one launch.

Both launch one HIP kernel on torch's current stream (no host sync, no device
value read), so the engine's graph capture of the decode step takes them
unchanged.  There is no fallback: without the HIP library every call raises.
"""

from __future__ import annotations

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
    """K splits of ``linear_partials`` for x [rows, k] @ W[n, k].T (a power of two).

    The plan lives in the library (qf_linear_splits) so C callers get the same
    one; compare engine/kernels/skinny_gemm.py:86-91, which ignores rows.
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
