"""Host-side checks of the drop-in surface (no GPU):

* the reference engine's ``from kernels.<module> import <name>`` statements
  (engine/decode_step.py:18-19, engine/engine.py:8, engine/prefill.py:28-29,
  engine/qk_norm_rope.py:7, engine/flash_decode.py:49) resolve to this
  package's modules when ``starter_amd/`` is on ``sys.path``, as the unchanged
  engine puts its own directory there;
* ``DecodeQKNormRoPE`` shares its wrapped attention's parameters (row views of
  one packed Q|K|V tensor) and, off the GPU, is exactly the model's own
  forward (the check of tests/test_qk_norm_rope.py:58-76 in the reference).
"""

from __future__ import annotations

import subprocess
import sys
import textwrap
from pathlib import Path
from unittest import mock

import torch
from transformers import Qwen3Config, Qwen3ForCausalLM

from starter_amd import modules

ROOT = Path(__file__).resolve().parents[1]

#: Every name the reference engine and its tests import from ``kernels``.
ENGINE_IMPORTS = {
    "kernels.decode_fused": ("add_rms_norm", "qkv_norm_rope_cache", "silu_mul", "MAX_BLOCK"),
    "kernels.skinny_gemm": ("linear_partials", "linear_silu_mul", "supports", "split_count",
                            "MAX_ROWS", "BN", "BK"),
    "kernels.rmsnorm": ("rms_norm", "MAX_BLOCK"),
    "kernels.prefill": ("prefill_qkv",),
    "kernels.qk_norm_rope": ("qk_norm_rope",),
    "kernels.small_query_attention": ("SmallQueryAttention", "partition_keys", "QUERY_TILE",
                                      "MAX_SPLITS"),
}


def tiny(**overrides):
    """The reference test model (tests/test_qk_norm_rope.py:29-37)."""
    cfg = dict(vocab_size=127, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
               num_attention_heads=4, num_key_value_heads=2, head_dim=128,
               max_position_embeddings=32768, rope_theta=5_000_000, tie_word_embeddings=True,
               sliding_window=None)
    cfg.update(overrides)
    config = Qwen3Config(**cfg)
    config._attn_implementation = "sdpa"
    return Qwen3ForCausalLM(config).eval()


def test_engine_import_path_resolves_to_this_package():
    """In a fresh interpreter with only ``starter_amd/`` added (no ``starter_amd``
    package import), every ``kernels.*`` name the engine imports exists and
    comes from ``starter_amd/kernels``; no Triton is imported."""
    script = textwrap.dedent(f"""
        import importlib, sys
        sys.path.insert(0, {str(ROOT / 'starter_amd')!r})
        wanted = {ENGINE_IMPORTS!r}
        for name, symbols in wanted.items():
            module = importlib.import_module(name)
            assert module.__file__.startswith({str(ROOT / 'starter_amd' / 'kernels')!r}), module.__file__
            for symbol in symbols:
                assert hasattr(module, symbol), (name, symbol)
        assert "triton" not in sys.modules, "a kernels module imported triton"
        assert "starter_amd" not in sys.modules
        print("ok")
    """)
    out = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                         cwd="/", timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().endswith("ok")


@torch.inference_mode()
def test_adapter_shares_weights_and_falls_back_off_gpu():
    torch.manual_seed(0)
    model = tiny()
    native = model.model.layers[0].self_attn
    names = set(native.state_dict())
    fused = modules.DecodeQKNormRoPE(native)
    assert not fused.training
    assert set(fused.state_dict()) == names == set(native.state_dict())
    params = dict(fused.named_parameters())
    for name, param in native.named_parameters():
        assert params[name] is param
    # q/k/v weights are row ranges of the packed tensor (no second copy).
    base = fused.qkv_weight.data_ptr()
    rows = [fused.q_proj.weight, fused.k_proj.weight, fused.v_proj.weight]
    offsets = [(w.data_ptr() - base) // w.element_size() for w in rows]
    assert offsets == [0, 4 * 128 * 256, 6 * 128 * 256]
    for length in (1, 7):
        x = torch.randn(2, length, 256)
        pos = torch.arange(length).unsqueeze(0)
        emb = model.model.rotary_emb(x, pos)
        for mask in (None, torch.ones(1, 1, length, length, dtype=torch.bool)):
            expected = native(x, emb, mask)[0]
            with mock.patch.object(modules, "qk_norm_rope",
                                   side_effect=AssertionError("must fall back on the CPU")):
                actual = fused(x, emb, mask)[0]
            torch.testing.assert_close(actual, expected, rtol=0, atol=0)


@torch.inference_mode()
def test_install_swaps_every_module():
    torch.manual_seed(1)
    model = modules.install(tiny())
    base = model.model
    assert isinstance(base.embed_tokens, modules.FusedEmbedding)
    assert base.embed_tokens.weight is model.lm_head.weight       # the tie is kept
    assert isinstance(base.norm, modules.FusedRMSNorm)
    for layer in base.layers:
        assert isinstance(layer.self_attn, modules.DecodeQKNormRoPE)
        assert isinstance(layer.self_attn.q_norm, modules.FusedRMSNorm)
        assert isinstance(layer.mlp, modules.PackedMLP)
        assert isinstance(layer.input_layernorm, modules.FusedRMSNorm)
