"""MI355X (gfx950) fused layer kernels of the Qwen3-4B decode engine.

``starter_amd.kernels`` holds the drop-in replacements of the reference
engine's ``kernels`` package (rmsnorm, qk_norm_rope, decode_fused, prefill)
plus ``embedding`` and ``rotary``; ``starter_amd.modules`` the Transformers
module adapters.  The kernels live in ``kernels/libqwen_fused.so``, built from
``csrc/*.hip`` by ``python -m starter_amd.build``.
"""
