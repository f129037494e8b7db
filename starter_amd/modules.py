"""Module adapters that put the HIP kernels inside a Transformers Qwen3 model.

* ``FusedRMSNorm`` - engine/engine.py:13-20: wraps a Qwen3RMSNorm's weight and
  epsilon and calls ``kernels.rmsnorm.rms_norm``.
* ``PackedMLP`` - engine/mlp.py:8-21: one packed ``[2I, H]`` gate/up weight;
  on CUDA bf16 the activation is the fused ``silu_mul`` kernel on the packed
  projection, elsewhere it is the reference module's own ``act_fn(gate) * up``.
* ``DecodeQKNormRoPE`` - engine/qk_norm_rope.py:10-71: a ``Qwen3Attention``
  whose single-token decode forward runs the per-head Q/K RMSNorm and the
  rotary embedding as one ``kernels.qk_norm_rope`` launch; every other call
  (prefill, CPU, training, unusual rotary layouts) is the model's own forward.
* ``FusedEmbedding`` - embedding gather that shares ``embed_tokens.weight``.
* ``install(model)`` - the module swaps ``Engine.__init__`` performs
  (engine/engine.py:39-47) for norms, MLPs, attention and the embedding.
"""

from __future__ import annotations

import copy

import torch
from torch import nn
from torch.nn import functional as F

from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention, eager_attention_forward

from .engine import _pack_rows
from .kernels.decode_fused import silu_mul
from .kernels.embedding import FusedEmbedding
from .kernels.qk_norm_rope import HEAD, qk_norm_rope
from .kernels.rmsnorm import rms_norm

__all__ = ["FusedRMSNorm", "PackedMLP", "DecodeQKNormRoPE", "FusedEmbedding", "install"]


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


class DecodeQKNormRoPE(Qwen3Attention):
    """``Qwen3Attention`` with the decode-step Q/K norm + RoPE fused.

    Adopts the wrapped attention's whole instance state - its submodules,
    parameters, buffers and configuration attributes, whatever this
    transformers version gives a ``Qwen3Attention`` - so no weight is
    allocated or initialised.  The q, k and v projections are then packed
    into one ``qkv_weight`` ``[(Hq + 2 Hkv) * 128, H]`` by the engine's own
    row packer, so the three modules read row ranges of it and the state dict,
    the prefill path and the fused decode step share one copy
    (engine/qk_norm_rope.py:10-30).
    """

    @torch.no_grad()
    def __init__(self, reference):
        nn.Module.__init__(self)
        # new containers, same members: swapping a module on one adapter does
        # not reach back into the wrapped attention
        for key, value in vars(reference).items():
            self.__dict__[key] = copy.copy(value) if isinstance(value, dict) else value
        self.qkv_weight = _pack_rows(self.q_proj, self.k_proj, self.v_proj)

    def _fused(self, hidden_states, cos, sin, cache, kwargs) -> bool:
        """True when the one-token kernel applies.  Reads shapes, dtypes and
        flags only (no device values), so the decision is capturable; the
        rules follow engine/qk_norm_rope.py:37-51, except that a missing
        attention mask does not force the fallback (transformers 5 passes
        none for an unpadded single-token step under SDPA)."""
        return not (
            hidden_states.ndim != 3 or hidden_states.shape[1] != 1
            or not hidden_states.is_cuda or hidden_states.dtype != torch.bfloat16
            or self.head_dim != HEAD or self.training
            or getattr(cache, "prefilling", False)
            or kwargs.get("output_attentions", False)
            or self.config._attn_implementation not in ("sdpa", "eager", "starter_decode_gqa")
            or cos.ndim != 3 or cos.shape != sin.shape
            or cos.shape[0] not in (1, hidden_states.shape[0])
            or tuple(cos.shape[1:]) != (1, HEAD)
            or cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16
            or any(m.bias is not None for m in (self.q_proj, self.k_proj, self.v_proj))
        )

    def forward(self, hidden_states, position_embeddings, attention_mask,
                past_key_values=None, **kwargs):
        # transformers 4.x passes the cache as ``past_key_value``.
        legacy = kwargs.pop("past_key_value", None)
        if past_key_values is None:
            past_key_values = legacy
        cos, sin = position_embeddings
        if not self._fused(hidden_states, cos, sin, past_key_values, kwargs):
            return super().forward(hidden_states, position_embeddings, attention_mask,
                                   past_key_values=past_key_values, **kwargs)
        batch = hidden_states.shape[0]
        nq = self.q_proj.weight.shape[0] // HEAD
        nk = self.k_proj.weight.shape[0] // HEAD
        # One packed projection; q, k and v are [B, H, 1, 128] views of its rows.
        qkv = F.linear(hidden_states, self.qkv_weight).view(batch, nq + 2 * nk, 1, HEAD)
        q, k, v = qkv[:, :nq], qkv[:, nq:nq + nk], qkv[:, nq + nk:]
        q, k = qk_norm_rope(q, k, self.q_norm.weight, self.k_norm.weight, cos, sin,
                            self.q_norm.variance_epsilon, self.k_norm.variance_epsilon)
        if past_key_values is not None:
            # transformers 4.x's StaticCache writes the slots named by
            # cache_position and, without it, every slot (engine/qk_norm_rope.py:
            # 64-66 passes the same three); transformers 5 layers ignore them
            k, v = past_key_values.update(k, v, self.layer_idx, {
                "sin": sin, "cos": cos, "cache_position": kwargs.get("cache_position")})
        interface = ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
                                                          eager_attention_forward)
        output, weights = interface(self, q, k, v, attention_mask, dropout=0.0,
                                    scaling=self.scaling, sliding_window=self.sliding_window,
                                    **kwargs)
        return self.o_proj(output.reshape(batch, 1, -1).contiguous()), weights


def install(model):
    """Swap a Qwen3ForCausalLM's norms, MLPs, attention and embedding for the
    fused modules (the swaps of engine/engine.py:39-47)."""
    base = model.model
    base.embed_tokens = FusedEmbedding(base.embed_tokens)
    base.norm = FusedRMSNorm(base.norm)
    for layer in base.layers:
        layer.input_layernorm = FusedRMSNorm(layer.input_layernorm)
        layer.post_attention_layernorm = FusedRMSNorm(layer.post_attention_layernorm)
        layer.self_attn.q_norm = FusedRMSNorm(layer.self_attn.q_norm)
        layer.self_attn.k_norm = FusedRMSNorm(layer.self_attn.k_norm)
        layer.mlp = PackedMLP(layer.mlp)
        layer.self_attn = DecodeQKNormRoPE(layer.self_attn)
    return model
