"""Drop-in replacements for the reference engine's ``kernels`` package.

The modules keep the reference's import paths (``kernels.rmsnorm``,
``kernels.qk_norm_rope``, ``kernels.decode_fused``, ``kernels.prefill``) and
add ``kernels.embedding`` and ``kernels.rotary``.  Every function runs a
hand-written gfx950 HIP kernel from ``libqwen_fused.so`` through ctypes; there
is no Triton and no fallback.  The package uses only relative imports, so it
works both as ``starter_amd.kernels`` and, with ``starter_amd/`` on
``sys.path``, as the engine's top-level ``kernels`` package.
"""
