"""Module adapters that put the HIP kernels inside a Transformers Qwen3 model.

* ``FusedRMSNorm`` - engine/engine.py:13-20: wraps a Qwen3RMSNorm's weight and
  epsilon and calls ``kernels.rmsnorm.rms_norm``.
* ``PackedMLP`` - engine/mlp.py:8-21: one packed ``[2I, H]`` gate/up weight;
  on CUDA bf16 the activation is the fused ``silu_mul`` kernel on the packed
  projection, elsewhere it is the reference module's own ``act_fn(gate) * up``.
* ``FusedEmbedding`` - embedding gather that shares ``embed_tokens.weight``.
* ``install(model)`` - the module swaps ``Engine.__init__`` performs
  (engine/engine.py:39-46) for norms, MLPs and the embedding.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F

from .kernels.decode_fused import silu_mul
from .kernels.embedding import FusedEmbedding
from .kernels.rmsnorm import rms_norm

__all__ = ["FusedRMSNorm", "PackedMLP", "FusedEmbedding", "install"]


class FusedRMSNorm(nn.Module):
    def __init__(self, reference):
        super().__init__()
        self.weight = reference.weight
        self.variance_epsilon = reference.variance_epsilon

    def forward(self, x):
        return rms_norm(x, self.weight, self.variance_epsilon)


def _is_silu(act) -> bool:
    return isinstance(act, nn.SiLU) or type(act).__name__ in ("SiLUActivation", "SiLU")


class PackedMLP(nn.Module):
    @torch.no_grad()
    def __init__(self, reference):
        super().__init__()
        self.gate_up_weight = nn.Parameter(
            torch.cat((reference.gate_proj.weight, reference.up_proj.weight)),
            requires_grad=False,
        )
        self.down_proj = reference.down_proj
        self.act_fn = reference.act_fn

    def forward(self, x):
        projected = F.linear(x, self.gate_up_weight)
        if projected.is_cuda and projected.dtype == torch.bfloat16 and _is_silu(self.act_fn):
            width = projected.shape[-1]
            hidden = silu_mul(projected.reshape(-1, width)).view(*projected.shape[:-1], width // 2)
            return self.down_proj(hidden)
        gate, up = projected.chunk(2, dim=-1)
        return self.down_proj(self.act_fn(gate) * up)


def install(model):
    """Swap a Qwen3ForCausalLM's norms, MLPs and embedding for the fused modules."""
    base = model.model
    base.embed_tokens = FusedEmbedding(base.embed_tokens)
    base.norm = FusedRMSNorm(base.norm)
    for layer in base.layers:
        layer.input_layernorm = FusedRMSNorm(layer.input_layernorm)
        layer.post_attention_layernorm = FusedRMSNorm(layer.post_attention_layernorm)
        layer.self_attn.q_norm = FusedRMSNorm(layer.self_attn.q_norm)
        layer.self_attn.k_norm = FusedRMSNorm(layer.self_attn.k_norm)
        layer.mlp = PackedMLP(layer.mlp)
    return model
