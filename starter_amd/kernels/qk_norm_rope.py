"""BF16 Q/K head RMSNorm plus RoPE for a single decode token, on gfx950 HIP.

Drop-in for ``engine/kernels/qk_norm_rope.py`` (jadenpxrk/starter): same
signature, shape rules, ``ValueError`` conditions and fresh contiguous outputs.
"""

from __future__ import annotations

import torch

from . import _lib

HEAD = 128


def _rows_view(t: torch.Tensor):
    """(tensor, batch_stride, head_stride) of a [B, H, 1, 128] operand whose
    head rows are 16-byte aligned, copying only when they are not (the
    reference always copies, engine/kernels/qk_norm_rope.py:63)."""
    if (t.stride(-1) != 1 or not _lib.aligned(t) or t.stride(0) % 8 or t.stride(1) % 8):
        t = t.contiguous()
    return t, t.stride(0), t.stride(1)


def qk_norm_rope(q, k, q_weight, k_weight, cos, sin, q_eps, k_eps):
    """One-token Q/K head RMSNorm + RoPE: returns new contiguous bf16 Q and K
    of shape ``[B, H, 1, 128]``.

    ``q`` and ``k`` (bf16 ``[B, H, 1, 128]``) may be strided views, such as
    head slices of one packed projection; they are read in place when their
    head rows are 16-byte aligned.  ``q_weight`` / ``k_weight`` are the
    ``[128]`` gains; ``cos`` / ``sin`` are the rotary rows the model already
    computed, ``[1, 1, 128]`` (shared) or ``[B, 1, 128]`` (per sequence).
    Nothing is written to the inputs.  Contract of
    engine/kernels/qk_norm_rope.py:47-73.
    """
    batch = q.shape[0]
    if (q.ndim != 4 or k.ndim != 4 or tuple(q.shape[2:]) != (1, HEAD)
            or tuple(k.shape[2:]) != (1, HEAD) or k.shape[0] != batch
            or cos.shape != sin.shape or cos.ndim != 3
            or cos.shape[0] not in (1, batch) or tuple(cos.shape[1:]) != (1, HEAD)
            or tuple(q_weight.shape) != (HEAD,) or tuple(k_weight.shape) != (HEAD,)):
        raise ValueError("Unsupported Q/K or rotary shape")
    inputs = (q, k, q_weight, k_weight, cos, sin)
    if not q.is_cuda or any(t.device != q.device or t.dtype != torch.bfloat16 for t in inputs):
        raise ValueError("Q/K norm-RoPE requires BF16 tensors on one CUDA device")
    nq, nk = q.shape[1], k.shape[1]
    oq = torch.empty((batch, nq, 1, HEAD), dtype=torch.bfloat16, device=q.device)
    ok = torch.empty((batch, nk, 1, HEAD), dtype=torch.bfloat16, device=q.device)
    if nq < 1 or nk < 1:
        raise ValueError("Q/K need at least one head each")
    if batch == 0:
        return oq, ok
    q, q_bs, q_hs = _rows_view(q)
    k, k_bs, k_hs = _rows_view(k)
    q_weight, k_weight = q_weight.contiguous(), k_weight.contiguous()
    cos, sin = cos.contiguous(), sin.contiguous()
    cs_bs = 0 if cos.shape[0] == 1 else cos.stride(0)
    _lib.call("qf_qk_norm_rope", q.data_ptr(), k.data_ptr(), batch, nq, nk, q_bs, q_hs, k_bs,
              k_hs, q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(),
              cs_bs, float(q_eps), float(k_eps), oq.data_ptr(), ok.data_ptr(),
              _lib.stream(q.device))
    return oq, ok
