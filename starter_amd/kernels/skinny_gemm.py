"""Stand-in for the reference's split-K decode projections (no Triton).

``engine/decode_step.py:19-30`` imports ``linear_partials``, ``linear_silu_mul``
and ``supports`` from ``kernels.skinny_gemm`` and calls the first two only when
``supports()`` accepts a shape.  The reference's versions are Triton GEMMs
(``engine/kernels/skinny_gemm.py:28-121``) - a dense contraction outside this
build's memory-bound kernels.  This module keeps the import working with the
same names and a static shape rule that declines every shape, so the engine
takes its own ``F.linear`` path (hipBLASLt on ROCm) followed by the fused
``add_rms_norm`` / ``qkv_norm_rope_cache`` / ``silu_mul`` kernels - the path the
reference takes for any shape its rule does not support.
"""

from __future__ import annotations

#: Decode row limit of the reference's rule (engine/kernels/skinny_gemm.py:22).
MAX_ROWS = 64


def supports(x, weight, pairs=False) -> bool:
    """Static shape rule: no shape is served by a split-K kernel here."""
    return False


def _unsupported(*_args, **_kwargs):
    raise ValueError("split-K decode projections are not provided by this build; "
                     "supports() is False for every shape")


def linear_partials(x, weight):
    """Never reached while supports() is False."""
    _unsupported()


def linear_silu_mul(x, gate_up_weight):
    """Never reached while supports() is False."""
    _unsupported()
