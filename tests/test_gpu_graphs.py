"""HIP-graph capture of the kernels and the module adapters on the GPU.

The wrappers launch on torch's current stream with no host synchronisation
or allocation outside torch, so a decode or prefill step containing them can
be captured (engine/decode.py:130-148, engine/prefill.py:79-96).  Each graph
is replayed several times with new inputs and positions, with eager work and
synchronisations between replays, and every replay is checked against the
oracle; output addresses must stay fixed (tests/test_decode_step.py:336-379,
tests/test_qk_norm_rope.py:177-202, tests/test_prefill.py:525-548 of the
reference).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn
from torch.nn import functional as F

from conftest import O, assert_bf16_close, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd import modules  # noqa: E402
from starter_amd.kernels.decode_fused import add_rms_norm, qkv_norm_rope_cache, silu_mul  # noqa: E402
from starter_amd.kernels.embedding import FusedEmbedding, embedding  # noqa: E402
from starter_amd.kernels.prefill import prefill_qkv  # noqa: E402
from starter_amd.kernels.qk_norm_rope import qk_norm_rope  # noqa: E402
from starter_amd.kernels.rmsnorm import rms_norm  # noqa: E402
from starter_amd.kernels.rotary import default_inv_freq, rope_tables  # noqa: E402

DEV = "cuda"
INV_FREQ = default_inv_freq(5_000_000, 128)


def capture(fn, warmups=3):
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(warmups):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outputs = fn()
    torch.cuda.synchronize()
    return graph, outputs


@torch.inference_mode()
def test_decode_kernels_graph_replay_follows_position_and_inputs():
    torch.manual_seed(14)
    capacity = 641
    cos, sin = rope_tables(INV_FREQ, capacity, device=DEV)
    qkv = torch.randn(3, 48 * 128, device=DEV).to(torch.bfloat16)
    qw = torch.randn(128, device=DEV).to(torch.bfloat16)
    kw = torch.randn(128, device=DEV).to(torch.bfloat16)
    pos = torch.tensor([0], device=DEV)
    keys = torch.zeros(3, 8, capacity, 128, dtype=torch.bfloat16, device=DEV)
    values = keys.clone()
    x = torch.randn(3, 2560, device=DEV).to(torch.bfloat16)
    y = torch.randn_like(x)
    w = torch.randn(2560, device=DEV).to(torch.bfloat16)
    gate_up = torch.randn(3, 2 * 9728, device=DEV).to(torch.bfloat16)
    table = torch.randn(500, 2560, device=DEV).to(torch.bfloat16)
    ids = torch.randint(0, 500, (3,), device=DEV)
    qm = torch.randn(3, 32, 1, 128, device=DEV).to(torch.bfloat16)
    km = torch.randn(3, 8, 1, 128, device=DEV).to(torch.bfloat16)
    cs_rows = torch.empty(3, 1, 128, dtype=torch.bfloat16, device=DEV)
    sn_rows = torch.empty_like(cs_rows)

    def step():
        return (qkv_norm_rope_cache(qkv, qw, kw, 1e-6, 1e-6, cos, sin, pos, keys, values),
                *add_rms_norm(x, y, w, 1e-6), silu_mul(gate_up), embedding(ids, table),
                rms_norm(x, w, 1e-6), *qk_norm_rope(qm, km, qw, kw, cs_rows, sn_rows, 1e-6, 3e-6))

    cs_rows.copy_(cos[:3].view(3, 1, 128))
    sn_rows.copy_(sin[:3].view(3, 1, 128))
    graph, outputs = capture(step)
    pointers = [t.data_ptr() for t in outputs]
    for position in (1, 300, 640, 7, 7):
        qkv.normal_(); x.normal_(); y.normal_(); gate_up.normal_(); qm.normal_(); km.normal_()
        ids.random_(0, 500)
        keys.zero_(); values.zero_()
        pos.fill_(position)
        rows = torch.tensor([position, (position * 7) % capacity, 3], device=DEV)
        cs_rows.copy_(cos[rows].view(3, 1, 128)); sn_rows.copy_(sin[rows].view(3, 1, 128))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eq, ek, ev = O.qkv_norm_rope_cache(bits(qkv), bits(qw), bits(kw), 1e-6, 1e-6, bits(cos),
                                           bits(sin), position,
                                           np.zeros(keys.shape, np.uint16),
                                           np.zeros(keys.shape, np.uint16))
        assert_bits_exact(outputs[0], eq, what=f"q @ {position}")
        assert_bits_exact(keys, ek)
        assert np.array_equal(bits(values), ev)
        e_total, e_normed = O.add_rms_norm(bits(x), bits(y), bits(w), 1e-6)
        assert np.array_equal(bits(outputs[1]), e_total)
        assert_bits_exact(outputs[2], e_normed)
        assert_bf16_close(outputs[3], O.silu_mul(bits(gate_up)), min_exact=0.999)
        assert torch.equal(outputs[4], F.embedding(ids, table))
        assert_bits_exact(outputs[5], O.rms_norm(bits(x), bits(w), 1e-6))
        mq, mk = O.qk_norm_rope(bits(qm)[:, :, 0], bits(km)[:, :, 0], bits(qw), bits(kw),
                                bits(cs_rows), bits(sn_rows), 1e-6, 3e-6)
        assert_bits_exact(bits(outputs[6])[:, :, 0], mq)
        assert_bits_exact(bits(outputs[7])[:, :, 0], mk)
        assert pointers == [t.data_ptr() for t in outputs]


@torch.inference_mode()
def test_prefill_graph_replay_updates_every_prompt_slot():
    b, t, c = 2, 17, 25
    p = torch.randn(b * t, 8 * 128, device=DEV).to(torch.bfloat16)  # nq 4, nk 2
    qw = torch.ones(128, dtype=torch.bfloat16, device=DEV)
    kw = qw.clone()
    cos, sin = rope_tables(INV_FREQ, c, device=DEV)
    k = torch.full((b, 2, c, 128), 33.0, dtype=torch.bfloat16, device=DEV)
    v = k.clone()
    graph, q = capture(lambda: prefill_qkv(p, qw, kw, 1e-6, 1e-6, cos, sin, k, v, t), warmups=2)
    addresses = [a.data_ptr() for a in (q, k, v)]
    for _ in range(3):
        p.normal_(); k.fill_(33); v.fill_(-41)
        before_k, before_v = bits(k), bits(v)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eq, ek, ev = O.prefill_qkv(bits(p), bits(qw), bits(kw), 1e-6, 1e-6, bits(cos), bits(sin),
                                   before_k, before_v, t)
        assert_bits_exact(q, eq)
        assert_bits_exact(k, ek)
        assert np.array_equal(bits(v), ev)
        assert addresses == [a.data_ptr() for a in (q, k, v)]


# ------------------------------------------------------------- module adapters

@torch.inference_mode()
def test_module_adapters_match_the_reference_modules():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(5)
    cfg = Qwen3Config(vocab_size=127, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=128, max_position_embeddings=32768, rope_theta=5_000_000,
                      tie_word_embeddings=True)
    model = Qwen3ForCausalLM(cfg).eval().to(DEV, torch.bfloat16)
    layer = model.model.layers[0]
    x = torch.randn(2, 7, 256, device=DEV).to(torch.bfloat16)
    reference_mlp = layer.mlp
    expected = reference_mlp(x)
    packed = modules.PackedMLP(reference_mlp)
    with torch.no_grad():
        hidden = F.linear(x, packed.gate_up_weight)
    gate, up = hidden.chunk(2, dim=-1)
    exact_chain = packed.down_proj(F.silu(gate) * up)
    got = packed(x)
    torch.testing.assert_close(got, exact_chain, rtol=2e-2, atol=2e-3)
    torch.testing.assert_close(got, expected, rtol=3e-2, atol=3e-2)
    norm = layer.input_layernorm
    torch.testing.assert_close(modules.FusedRMSNorm(norm)(x), norm(x), rtol=1e-2, atol=1e-2)
    qn = layer.self_attn.q_norm
    q = torch.randn(2, 4, 7, 128, device=DEV).to(torch.bfloat16)
    torch.testing.assert_close(modules.FusedRMSNorm(qn)(q), qn(q), rtol=1e-2, atol=1e-2)
    ids = torch.randint(0, 127, (2, 7), device=DEV)
    tied = model.lm_head.weight is model.model.embed_tokens.weight
    emb = FusedEmbedding(model.model.embed_tokens)
    assert torch.equal(emb(ids), model.model.embed_tokens(ids))
    modules.install(model)
    assert isinstance(model.model.embed_tokens, FusedEmbedding)
    assert (model.lm_head.weight is model.model.embed_tokens.weight) == tied
    assert isinstance(model.model.layers[1].mlp, modules.PackedMLP)
    assert isinstance(model.model.norm, modules.FusedRMSNorm)
