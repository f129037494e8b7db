"""LM head fused with greedy token selection (gfx950).

The reference engine ends every step with ``F.linear(normed, lm_head.weight)``
and ``logits.argmax(-1)`` (engine/decode_step.py:64, engine/decode.py:93,106);
OPTIMIZATION_GUIDE.md:213 describes fusing them.  ``lm_head_argmax`` does it
in one vocabulary-tiled pass over the (tied) weight: bf16 logits rounded as
F.linear's output is, the argmax taken over them with the lowest index on
exact ties (torch.argmax's rule), per-tile candidates reduced by a second
small launch.  No host sync; capturable.  There is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib

MAX_ROWS = 64


def supports(x, weight) -> bool:
    """Static rule: contiguous bf16 CUDA x [1..64, K] and W [V, K], K % 64 == 0,
    V % 16 == 0, 16-byte aligned starts."""
    return (x.ndim == 2 and weight.ndim == 2 and x.shape[1] == weight.shape[1]
            and x.is_cuda and weight.device == x.device
            and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and x.is_contiguous() and weight.is_contiguous()
            and 1 <= x.shape[0] <= MAX_ROWS and x.shape[1] % 64 == 0 and weight.shape[0] % 16 == 0
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


def lm_head_argmax(x, weight, logits: bool = False, tokens=None, advance=None):
    """Greedy tokens int64 [M] of bf16 logits x @ weight.T; with ``logits=True``
    also returns those bf16 logits [M, V].  ``tokens`` may be a contiguous
    int64 [M] tensor on x's device to write the tokens into.  ``advance``:
    optional (position int64 [1], lengths int32 [L]) device tensors that the
    same launches increment by one (the decode step's state advance)."""
    if not supports(x, weight):
        raise ValueError("expected contiguous BF16 CUDA x[M<=64,K], W[V,K] with K % 64 == 0, V % 16 == 0")
    rows, k = x.shape
    vocab = weight.shape[0]
    blocks = _lib.lib().qf_lm_head_blocks(vocab)
    candidates = torch.empty((rows, blocks, 2), dtype=torch.int32, device=x.device)
    if tokens is None:
        tokens = torch.empty((rows,), dtype=torch.int64, device=x.device)
    elif (tokens.shape != (rows,) or tokens.dtype != torch.int64 or tokens.device != x.device
          or not tokens.is_contiguous()):
        raise ValueError("tokens must be a contiguous int64 [M] tensor on x's device")
    out = torch.empty((rows, vocab), dtype=torch.bfloat16, device=x.device) if logits else None
    if advance is None:
        _lib.call("qf_lm_head_argmax", x.data_ptr(), rows, k, weight.data_ptr(), vocab,
                  candidates.data_ptr(), tokens.data_ptr(), _lib.ptr(out), _lib.stream(x.device))
    else:
        position, lengths = advance
        for t, dtype in ((position, torch.int64), (lengths, torch.int32)):
            if t.dtype != dtype or t.device != x.device or not t.is_contiguous():
                raise ValueError("advance takes contiguous int64 position and int32 lengths on x's device")
        if position.numel() != 1:
            raise ValueError("position must hold one element")
        _lib.call("qf_lm_head_argmax_advance", x.data_ptr(), rows, k, weight.data_ptr(), vocab,
                  candidates.data_ptr(), tokens.data_ptr(), _lib.ptr(out), position.data_ptr(),
                  lengths.data_ptr(), lengths.numel(), _lib.stream(x.device))
    return (tokens, out) if logits else tokens
