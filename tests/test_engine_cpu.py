"""Host-side pieces of the Engine harness on the CPU: weight packing follows
transformers' module layout, and the engine refuses to run without a GPU."""

from __future__ import annotations

import pytest
import torch
from transformers import Qwen3Config, Qwen3ForCausalLM

from starter_amd import engine

TINY = dict(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=128,
            max_position_embeddings=4096, rope_theta=5_000_000, tie_word_embeddings=True)


def test_pack_layer_row_order():
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(Qwen3Config(**TINY)).eval()
    layer = model.model.layers[1]
    packed = engine.pack_layer(layer)
    attn, mlp = layer.self_attn, layer.mlp
    assert packed.qkv.shape == ((4 + 2 * 2) * 128, 256)
    q, k, v = packed.qkv.split([4 * 128, 2 * 128, 2 * 128])
    assert torch.equal(q, attn.q_proj.weight) and torch.equal(k, attn.k_proj.weight)
    assert torch.equal(v, attn.v_proj.weight)
    gate, up = packed.gate_up.chunk(2)
    assert torch.equal(gate, mlp.gate_proj.weight) and torch.equal(up, mlp.up_proj.weight)
    assert torch.equal(packed.down, mlp.down_proj.weight) and torch.equal(packed.o, attn.o_proj.weight)
    assert packed.eps_q == attn.q_norm.variance_epsilon
    assert all(t.is_contiguous() for t in (packed.qkv, packed.gate_up, packed.o, packed.down))
    # the modules now read row ranges of the packed tensors (one copy in memory)
    size = packed.qkv.element_size()
    for w, start in ((attn.q_proj.weight, 0), (attn.k_proj.weight, 4 * 128),
                     (attn.v_proj.weight, 6 * 128)):
        assert w.data_ptr() == packed.qkv.data_ptr() + start * 256 * size
    assert mlp.gate_proj.weight.data_ptr() == packed.gate_up.data_ptr()
    assert mlp.up_proj.weight.data_ptr() == packed.gate_up.data_ptr() + 512 * 256 * size


def test_rotary_check():
    engine.check_rotary(Qwen3ForCausalLM(Qwen3Config(**TINY)))
    scaled = dict(TINY, rope_scaling={"rope_type": "yarn", "factor": 4.0,
                                      "original_max_position_embeddings": 4096})
    with pytest.raises(ValueError):
        engine.check_rotary(Qwen3ForCausalLM(Qwen3Config(**scaled)))


def test_engine_needs_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("this host has a GPU")
    with pytest.raises(RuntimeError):
        engine.Engine(config=Qwen3Config(**TINY))


def test_tuned_gemms_file_is_a_tunableop_table():
    """The recorded prefill solutions: TunableOp's CSV (validator lines, then
    op, shape key, solution, time) with one entry per shape."""
    from starter_amd.engine import TUNED_GEMMS
    lines = TUNED_GEMMS.read_text().splitlines()
    validators = [line.split(",") for line in lines if line.startswith("Validator,")]
    assert {v[1] for v in validators} >= {"PT_VERSION", "GCN_ARCH_NAME", "HIPBLASLT_VERSION"}
    assert any(v[1] == "GCN_ARCH_NAME" and v[2].startswith("gfx950") for v in validators)
    entries = [line.split(",") for line in lines if line and not line.startswith("Validator,")]
    assert entries and all(len(e) == 4 and e[0].startswith("GemmTunableOp_") for e in entries)
    assert len({e[1] for e in entries}) == len(entries)
    assert all(float(e[3]) > 0 for e in entries)
