"""ctypes binding of ``libqwen_fused.so`` (the C ABI of ``include/qwen_fused.h``).

torch is imported before the library is opened: the library was linked
against ``libamdhip64.so.7`` and the dynamic loader then reuses the HIP runtime
torch already mapped (same SONAME), so torch's streams and device pointers are
valid inside the library.

There is no fallback: if the library is missing or fails to load, every
kernel call raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY = Path(__file__).with_name("libqwen_fused.so")

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

#: Every entry point of include/qwen_fused.h with its ctypes signature.
SIGNATURES = {
    "qf_version": ([], _i32),
    "qf_error_string": ([_i32], ctypes.c_char_p),
    "qf_rms_norm": ([_vp, _i64, _i64, _i64, _i64, _i64, _vp, _f32, _vp, _vp], _i32),
    "qf_add_rms_norm": ([_vp, _vp, _i32, _vp, _i64, _i64, _f32, _vp, _vp, _vp], _i32),
    "qf_silu_mul": ([_vp, _i64, _i64, _vp, _vp], _i32),
    "qf_qk_norm_rope": ([_vp, _vp, _i64, _i32, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                         _i64, _f32, _f32, _vp, _vp, _vp], _i32),
    "qf_qkv_norm_rope_cache": ([_vp, _i32, _i64, _i32, _i32, _vp, _vp, _f32, _f32, _vp, _vp, _vp,
                                _i64, _vp, _vp, _vp, _vp], _i32),
    "qf_prefill_qkv": ([_vp, _i64, _i64, _i32, _i32, _vp, _vp, _f32, _f32, _vp, _vp, _i64, _vp,
                        _vp, _vp, _vp], _i32),
    "qf_prefill_attention": ([_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i64, _f32, _vp, _vp], _i32),
    "qf_embedding": ([_vp, _i64, _vp, _i64, _i64, _vp, _vp], _i32),
    "qf_rope_table": ([_vp, _i32, _vp, _i64, _i64, _vp, _vp, _vp], _i32),
    "qf_linear_splits": ([_i64, _i64, _i64], _i32),
    "qf_linear_partials": ([_vp, _i64, _i64, _vp, _i64, _i32, _vp, _vp], _i32),
    "qf_linear_partials_merged": ([_vp, _vp, _i32, _i64, _i32, _i32, _vp, _i64, _i32, _vp, _vp],
                                  _i32),
    "qf_linear_silu_mul": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp], _i32),
    "qf_row_supported": ([_i32, _i64, _i64], _i32),
    "qf_linear_rows": ([_vp, _i32, _i64, _vp, _i64, _vp, _vp], _i32),
    "qf_linear_residual": ([_vp, _i32, _i64, _vp, _i64, _vp, _vp, _vp, _vp], _i32),
    "qf_linear_normed": ([_vp, _vp, _vp, _f32, _i32, _i64, _vp, _i64, _vp, _vp], _i32),
    "qf_row_merged_supported": ([_i32, _i32, _i32, _i32, _i64], _i32),
    "qf_linear_residual_merged": ([_vp, _vp, _i32, _i32, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _vp],
                                  _i32),
    "qf_row_silu_supported": ([_i32, _i64, _i64], _i32),
    "qf_linear_silu_mul_normed": ([_vp, _vp, _vp, _f32, _i32, _i64, _vp, _i64, _vp, _vp], _i32),
    "qf_linear_partials_normed": ([_vp, _vp, _vp, _f32, _i64, _i64, _vp, _i64, _i32, _vp, _vp],
                                  _i32),
    "qf_linear_silu_mul_normed_tiled": ([_vp, _vp, _vp, _f32, _i64, _i64, _vp, _i64, _vp, _vp],
                                        _i32),
    "qf_attention_partition": ([_i64, _i64, _i32, _vp, _vp], _i32),
    "qf_attention_partition_aligned": ([_i64, _i64, _i32, _i32, _vp, _vp], _i32),
    "qf_decode_attention": ([_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i64, _f32, _i32, _i64, _vp, _vp,
                             _vp, _vp], _i32),
    "qf_decode_attention_qkv": ([_vp, _i32, _vp, _vp, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _i64, _i32, _i32, _i64, _f32, _i32, _i64, _vp, _vp, _vp, _vp],
                                _i32),
    "qf_lm_head_blocks": ([_i64], _i64),
    "qf_lm_head_argmax": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp], _i32),
    "qf_lm_head_argmax_advance": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _vp],
                                  _i32),
    "qf_lm_head_argmax_static": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp], _i32),
}

_handle: ctypes.CDLL | None = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """The loaded library, with argtypes/restype set for every entry point."""
    global _handle
    if _handle is None:
        with _lock:
            if _handle is None:
                if not LIBRARY.exists():
                    raise RuntimeError(
                        f"{LIBRARY} is not built: run `python -m starter_amd.build` "
                        "(there is no fallback implementation)")
                handle = ctypes.CDLL(str(LIBRARY))
                for name, (args, res) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.argtypes = args
                    fn.restype = res
                _handle = handle
    return _handle


def stream(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (graph-capturable)."""
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    """Invoke entry point ``name``; a nonzero status raises RuntimeError."""
    status = getattr(lib(), name)(*args)
    if status != 0:
        text = lib().qf_error_string(status).decode()
        raise RuntimeError(f"{name} failed: {text} (status {status})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def aligned(t: torch.Tensor) -> bool:
    """16-byte aligned start (the 128-bit vector paths need it)."""
    return t.data_ptr() % 16 == 0
