"""CPU ORACLE (test infrastructure only): numpy bindings of ``qf_oracle.c``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, always as the checker and never as the thing measured
or shipped.  bf16 tensors are exchanged as ``np.uint16`` bit patterns.

Every function follows the reference file:line cited in ``qf_oracle.c``.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import build as _build

_LIB = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

_SIGNATURES = {
    "or_bf16": ([_f32], ctypes.c_uint16),
    "or_f32": ([ctypes.c_uint16], _f32),
    "or_rms_norm": ([_vp, _i64, _i64, _vp, _f32, _vp, _vp], None),
    "or_add_rms_norm": ([_vp, _vp, _i32, _vp, _i64, _i64, _f32, _vp, _vp, _vp], None),
    "or_silu_mul": ([_vp, _i64, _i64, _vp], None),
    "or_qk_norm_rope": ([_vp, _vp, _i64, _i32, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                         _i64, _f32, _f32, _i32, _vp, _vp], None),
    "or_qkv_norm_rope_cache": ([_vp, _i32, _i64, _i32, _i32, _vp, _vp, _f32, _f32, _vp, _vp,
                                _i64, _i64, _i32, _vp, _vp, _vp], None),
    "or_prefill_qkv": ([_vp, _i64, _i64, _i32, _i32, _vp, _vp, _f32, _f32, _vp, _vp, _i64, _i32,
                        _vp, _vp, _vp], None),
    "or_embedding": ([_vp, _i64, _vp, _i64, _i64, _vp], None),
    "or_rope_table": ([_vp, _i32, _vp, _i64, _i64, _vp, _vp], None),
    "or_linear_partials": ([_vp, _i64, _i64, _vp, _i64, _i32, _vp], None),
    "or_linear_silu_mul": ([_vp, _i64, _i64, _vp, _i64, _vp], None),
    "or_prefill_attention": ([_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i64, ctypes.c_double, _vp,
                              _vp], None),
    "or_decode_attention": ([_vp, _vp, _vp, _vp, _i64, _i32, _i32, _i64, ctypes.c_double, _vp, _vp],
                            None),
    "or_lm_head_argmax": ([_vp, _i64, _i64, _vp, _i64, _vp, _vp], None),
}


def lib() -> ctypes.CDLL:
    """Load (building on first use) the oracle shared library."""
    global _LIB
    if _LIB is None:
        path = _build.LIBRARY
        if not path.exists():
            _build.build()
        handle = ctypes.CDLL(str(path))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = handle
    return _LIB


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_vp)


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


# ----------------------------------------------------------------- bf16 math

def bf16_bits(x) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even, NaN -> 0x7FC0 (vectorised)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), r)


def bf16_value(bits) -> np.ndarray:
    """bf16 bits -> exact f32 values."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 bit arrays (monotone integer map)."""
    def key(bits):
        s = np.asarray(bits, dtype=np.uint16).astype(np.int32)
        return np.where(s & 0x8000, 0x8000 - s, s)  # -0 and +0 both map to 0
    return np.abs(key(a_bits) - key(b_bits))


# ------------------------------------------------------------------ the ops

def rms_norm(x, weight, eps: float) -> np.ndarray:
    """engine/kernels/rmsnorm.py:39-62 on bf16 bits; last dimension normalised."""
    x = _u16(x)
    cols = x.shape[-1]
    rows = x.size // cols if cols else 0
    out = np.empty_like(x)
    scratch = np.empty(max(cols, 1), dtype=np.float32)
    lib().or_rms_norm(_p(x), rows, cols, _p(_u16(weight)), eps, _p(scratch), _p(out))
    return out


def add_rms_norm(residual, branch, weight, eps: float):
    """engine/kernels/decode_fused.py:140-158; branch is bf16 bits [R, C] or
    f32 split-K partials [S, R, C].  Returns (total, normed)."""
    residual = _u16(residual)
    rows, cols = residual.shape
    if branch.dtype == np.float32 and branch.ndim == 3:
        branch = np.ascontiguousarray(branch)
        splits = branch.shape[0]
    else:
        branch = _u16(branch)
        splits = 0
    total = np.empty_like(residual)
    normed = np.empty_like(residual)
    scratch = np.empty(max(cols, 1), dtype=np.float32)
    lib().or_add_rms_norm(_p(residual), _p(branch), splits, _p(_u16(weight)), rows, cols, eps,
                          _p(scratch), _p(total), _p(normed))
    return total, normed


def silu_mul(gate_up) -> np.ndarray:
    """engine/kernels/decode_fused.py:161-169 on a packed [rows, 2*cols] input."""
    gate_up = _u16(gate_up)
    rows, width = gate_up.shape
    cols = width // 2
    out = np.empty((rows, cols), dtype=np.uint16)
    lib().or_silu_mul(_p(gate_up), rows, cols, _p(out))
    return out


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, q_eps, k_eps, round_products=True):
    """engine/kernels/qk_norm_rope.py:47-73.  q [B, NQ, 128], k [B, NK, 128]
    bits; cos/sin [1 or B, 128].  Returns (oq, ok) shaped like q, k."""
    q, k = _u16(q), _u16(k)
    batch, nq, _ = q.shape
    nk = k.shape[1]
    cos, sin = _u16(cos).reshape(-1, 128), _u16(sin).reshape(-1, 128)
    cs_bs = 0 if cos.shape[0] == 1 else 128
    oq, ok = np.empty_like(q), np.empty_like(k)
    lib().or_qk_norm_rope(_p(q), _p(k), batch, nq, nk, nq * 128, 128, nk * 128, 128,
                          _p(_u16(q_weight)), _p(_u16(k_weight)), _p(cos), _p(sin), cs_bs,
                          q_eps, k_eps, int(round_products), _p(oq), _p(ok))
    return oq, ok


def qkv_norm_rope_cache(qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, position: int,
                        key_cache, value_cache, round_products=True):
    """engine/kernels/decode_fused.py:172-210.  qkv: bf16 bits [B, W] or f32
    partials [S, B, W].  Returns (q [B, NQ, 1, 128], key_cache', value_cache')
    where the caches are updated copies."""
    key_cache, value_cache = _u16(key_cache).copy(), _u16(value_cache).copy()
    batch, nk, capacity, head = key_cache.shape
    if qkv.dtype == np.float32 and qkv.ndim == 3:
        qkv = np.ascontiguousarray(qkv)
        splits = qkv.shape[0]
    else:
        qkv = _u16(qkv)
        splits = 0
    width = qkv.shape[-1]
    nq = width // head - 2 * nk
    q = np.empty((batch, nq, 1, head), dtype=np.uint16)
    lib().or_qkv_norm_rope_cache(_p(qkv), splits, batch, nq, nk, _p(_u16(q_weight)),
                                 _p(_u16(k_weight)), q_eps, k_eps, _p(_u16(cos)), _p(_u16(sin)),
                                 int(position), capacity, int(round_products), _p(q),
                                 _p(key_cache), _p(value_cache))
    return q, key_cache, value_cache


def prefill_qkv(qkv, q_weight, k_weight, q_eps, k_eps, cos, sin, key_cache, value_cache,
                length: int, round_products=True):
    """engine/kernels/prefill.py:66-96.  Returns (q [B, T, NQ, 128],
    key_cache', value_cache') with the caches updated copies."""
    key_cache, value_cache = _u16(key_cache).copy(), _u16(value_cache).copy()
    batch, nk, capacity, head = key_cache.shape
    qkv = _u16(qkv)
    nq = qkv.shape[1] // head - 2 * nk
    q = np.empty((batch, length, nq, head), dtype=np.uint16)
    lib().or_prefill_qkv(_p(qkv), batch, length, nq, nk, _p(_u16(q_weight)), _p(_u16(k_weight)),
                         q_eps, k_eps, _p(_u16(cos)), _p(_u16(sin)), capacity,
                         int(round_products), _p(q), _p(key_cache), _p(value_cache))
    return q, key_cache, value_cache


def embedding(ids, table) -> np.ndarray:
    """nn.Embedding lookup (engine/decode_step.py:38); out-of-range ids -> 0."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    table = _u16(table)
    vocab, cols = table.shape
    out = np.empty(ids.shape + (cols,), dtype=np.uint16)
    lib().or_embedding(_p(ids), ids.size, _p(table), vocab, cols, _p(out))
    return out


def rope_table(inv_freq, n_pos: int | None = None, positions=None, start: int = 0):
    """engine/decode.py:52-59 (Qwen3RotaryEmbedding.forward per slot).
    Returns (cos, sin) bits [n, 2*half]."""
    inv_freq = np.ascontiguousarray(inv_freq, dtype=np.float32)
    half = inv_freq.size
    if positions is not None:
        positions = np.ascontiguousarray(positions, dtype=np.int64)
        n_pos = positions.size
    cos = np.empty((n_pos, 2 * half), dtype=np.uint16)
    sin = np.empty_like(cos)
    lib().or_rope_table(_p(inv_freq), half, _p(positions), start, n_pos, _p(cos), _p(sin))
    return cos, sin


def default_inv_freq(theta: float, dim: int) -> np.ndarray:
    """Qwen3 default inverse frequencies 1 / theta**(2j/dim) in f32: the
    exponent is rounded to f32 as torch does (arange -> / dim), the power is
    evaluated in f64 and rounded once, then the f32 reciprocal is taken.
    torch's f32 pow is accurate to about one f32 ulp, so the model's buffer
    and this helper agree to within two f32 ulps."""
    e = (np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim)).astype(np.float32)
    p = np.power(np.float64(theta), e.astype(np.float64)).astype(np.float32)
    return (np.float32(1.0) / p).astype(np.float32)


__all__ = [name for name in dir() if not name.startswith("_") and name not in ("annotations", "ctypes", "np", "Path")]


def linear_partials(x, weight, splits: int) -> np.ndarray:
    """engine/kernels/skinny_gemm.py:28-46, 100-109: f32 [splits, M, N] partials of
    x [M, K] @ weight [N, K].T over K/splits-wide chunks (exactly rounded)."""
    x, weight = _u16(x), _u16(weight)
    m, k = x.shape
    n = weight.shape[0]
    if weight.shape[1] != k or splits < 1 or k % splits:
        raise ValueError("linear_partials: shapes disagree")
    out = np.empty((splits, m, n), dtype=np.float32)
    lib().or_linear_partials(_p(x), m, k, _p(weight), n, splits, _p(out))
    return out


def linear_silu_mul(x, gate_up) -> np.ndarray:
    """engine/kernels/skinny_gemm.py:49-72, 112-121: bf16 bits [M, N] of
    silu(bf16(x @ gate.T)) * bf16(x @ up.T) for a packed [2N, K] weight."""
    x, gate_up = _u16(x), _u16(gate_up)
    m, k = x.shape
    width = gate_up.shape[0]
    if gate_up.shape[1] != k or width % 2:
        raise ValueError("linear_silu_mul: shapes disagree")
    out = np.empty((m, width // 2), dtype=np.uint16)
    lib().or_linear_silu_mul(_p(x), m, k, _p(gate_up), width // 2, _p(out))
    return out


def decode_attention(q, k, v, used, scale: float) -> np.ndarray:
    """engine/kernels/small_query_attention.py:113-158 in float64: q bits
    [B, Hq, 1, 128], k/v bits [B, Hkv, C, 128], used int32 [B*Hkv].
    Returns bf16 bits [B, 1, Hq, 128]."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    used = np.ascontiguousarray(used, dtype=np.int32)
    batch, hq = q.shape[0], q.shape[1]
    hk, capacity = k.shape[1], k.shape[2]
    out = np.empty((batch, 1, hq, 128), dtype=np.uint16)
    scratch = np.empty(max(capacity, 1), dtype=np.float64)
    lib().or_decode_attention(_p(q), _p(k), _p(v), _p(used), batch, hq, hk, capacity, float(scale),
                              _p(scratch), _p(out))
    return out


def prefill_attention(q, k, v, length: int, scale: float) -> np.ndarray:
    """engine/prefill.py:13-23 in float64: causal attention of q bits
    [B, T, Hq, 128] over the first T slots of k/v bits [B, Hkv, C, 128].
    Returns bf16 bits [B, T, Hq, 128]."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    batch, hq = q.shape[0], q.shape[2]
    hk, capacity = k.shape[1], k.shape[2]
    if q.shape[1] != length or length > capacity or hq % hk:
        raise ValueError("prefill_attention: shapes disagree")
    out = np.empty_like(q)
    scratch = np.empty(max(length, 1), dtype=np.float64)
    lib().or_prefill_attention(_p(q), _p(k), _p(v), batch, length, hq, hk, capacity, float(scale),
                               _p(scratch), _p(out))
    return out


def lm_head_argmax(x, weight):
    """engine/decode_step.py:64 + argmax: (tokens int64 [M], bf16 logits bits
    [M, V]) with exactly rounded logits and first-maximum tie-breaking."""
    x, weight = _u16(x), _u16(weight)
    m, k = x.shape
    vocab = weight.shape[0]
    tokens = np.empty(m, dtype=np.int64)
    logits = np.empty((m, vocab), dtype=np.uint16)
    lib().or_lm_head_argmax(_p(x), m, k, _p(weight), vocab, _p(tokens), _p(logits))
    return tokens, logits
