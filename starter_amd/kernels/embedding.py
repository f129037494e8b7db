"""Token embedding gather on gfx950 HIP (bit-exact ``nn.Embedding`` lookup).

The engine calls ``base.embed_tokens(ids)`` (engine/decode_step.py:38,
engine/prefill.py:34, engine/decode.py:19).  ``FusedEmbedding`` replaces that
module while keeping the very same ``weight`` Parameter object, so the tie to
``lm_head.weight`` survives the swap.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _lib


def embedding(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``weight[ids]`` as a fresh contiguous tensor of shape ``ids.shape + (H,)``.

    Rows are copied bit for bit.  Unlike aten's gather, an id outside
    [0, vocab) is not a device assert: it yields a zero row.
    """
    if weight.ndim != 2 or not weight.is_cuda or weight.dtype != torch.bfloat16:
        raise ValueError("embedding table must be a 2-D BF16 CUDA tensor")
    if ids.dtype != torch.int64 or ids.device != weight.device:
        raise ValueError("ids must be int64 on the table's device")
    vocab, cols = weight.shape
    out = torch.empty((*ids.shape, cols), dtype=weight.dtype, device=weight.device)
    if ids.numel() == 0 or cols == 0:
        return out
    ids = ids.contiguous()
    weight = weight.contiguous()
    _lib.call("qf_embedding", ids.data_ptr(), ids.numel(), weight.data_ptr(), vocab, cols,
              out.data_ptr(), _lib.stream(weight.device))
    return out


class FusedEmbedding(nn.Module):
    """Stand-in for a Qwen3 ``embed_tokens`` module that shares its weight."""

    def __init__(self, reference: nn.Embedding):
        super().__init__()
        if getattr(reference, "max_norm", None) is not None:
            raise ValueError("max_norm embeddings are not supported")
        self.weight = reference.weight  # the same Parameter object: lm_head tie kept
        self.padding_idx = getattr(reference, "padding_idx", None)
        self.num_embeddings, self.embedding_dim = self.weight.shape

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return embedding(ids, self.weight)
