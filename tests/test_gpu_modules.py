"""The Transformers module path on the MI355X: a tiny Qwen3 with ``install()``
applied (fused norms, packed MLP with ``silu_mul``, the fused embedding and
``DecodeQKNormRoPE``), decoded token by token through the model's own forward
and KV cache, against the unmodified model.

Follows tests/test_qk_norm_rope.py:160-199 of the reference: same tiny model,
the shapes (3, 7, 5), (1, 1, 3) and (2, 13, 1), logits within rtol 0.03 /
atol 0.04 of the native bf16 model at every step, the candidate continuing
from its own tokens.  Prefill (more than one token) must not touch the Q/K
kernel and every single-token step must call it once per layer.
"""

from __future__ import annotations

import copy
from unittest import mock

import pytest
import torch
from transformers import DynamicCache, Qwen3Config, Qwen3ForCausalLM

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd import modules  # noqa: E402
from starter_amd.kernels.qk_norm_rope import qk_norm_rope  # noqa: E402


def tiny():
    cfg = Qwen3Config(vocab_size=127, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                      max_position_embeddings=32768, rope_theta=5_000_000,
                      tie_word_embeddings=True, sliding_window=None)
    cfg._attn_implementation = "sdpa"
    return Qwen3ForCausalLM(cfg).eval()


@pytest.fixture(scope="module")
def models():
    torch.manual_seed(7)
    native = tiny().cuda().bfloat16()
    candidate = modules.install(copy.deepcopy(native))
    return native, candidate


@pytest.mark.parametrize("batch,length,count", [(3, 7, 5), (1, 1, 3), (2, 13, 1)])
@torch.inference_mode()
def test_decode_through_modules_matches_native(models, batch, length, count):
    native, candidate = models
    layers = len(candidate.model.layers)
    prompt = torch.randint(0, 127, (batch, length), device="cuda")
    ours, theirs = DynamicCache(), DynamicCache()
    current = prompt
    for step in range(count):
        with mock.patch.object(modules, "qk_norm_rope", wraps=qk_norm_rope) as call:
            actual = candidate(input_ids=current, past_key_values=ours, use_cache=True,
                               logits_to_keep=1).logits
        # multi-token prefill keeps the model's own path; one-token steps
        # (including a one-token prompt) run the kernel once per layer
        assert call.call_count == (layers if current.shape[1] == 1 else 0)
        expected = native(input_ids=current, past_key_values=theirs, use_cache=True,
                          logits_to_keep=1).logits
        torch.testing.assert_close(actual, expected, rtol=0.03, atol=0.04)
        current = actual[:, -1].argmax(-1, keepdim=True)   # the candidate's own prefix
    assert ours.get_seq_length() == length + count - 1


@torch.inference_mode()
def test_single_token_attention_matches_native_module(models):
    """One layer's attention at T = 1 against the unfused module on the same
    cache contents, and the K/V rows it appends to the cache."""
    native, candidate = models
    torch.manual_seed(11)
    ours, theirs = DynamicCache(), DynamicCache()
    prompt = torch.randint(0, 127, (2, 9), device="cuda")
    candidate(input_ids=prompt, past_key_values=ours, use_cache=True)
    native(input_ids=prompt, past_key_values=theirs, use_cache=True)
    x = torch.randn(2, 1, 256, device="cuda", dtype=torch.bfloat16)
    pos = torch.full((1, 1), 9, device="cuda")
    emb = native.model.rotary_emb(x, pos)
    got = candidate.model.layers[0].self_attn(x, emb, None, past_key_values=ours)[0]
    want = native.model.layers[0].self_attn(x, emb, None, past_key_values=theirs)[0]
    torch.testing.assert_close(got, want, rtol=0.02, atol=0.02)
    # the packed projection may round differently from the separate ones
    # (hipBLASLt picks per output width), so the appended rows agree to the
    # bf16 tolerance rather than bit for bit
    for ours_t, theirs_t in ((ours.layers[0].keys, theirs.layers[0].keys),
                             (ours.layers[0].values, theirs.layers[0].values)):
        assert ours_t.shape[2] == theirs_t.shape[2] == 10
        torch.testing.assert_close(ours_t[:, :, -1], theirs_t[:, :, -1], rtol=0.02, atol=0.02)


@torch.inference_mode()
def test_decode_through_static_cache_matches_native(models):
    """The fixed-capacity cache the reference engine decodes into
    (engine/decode.py:7-12, a StaticCache subclass): four greedy steps after
    a 6-token prompt, and every one-token ``update`` receives the rotary rows
    and ``cache_position`` the reference adapter hands it
    (engine/qk_norm_rope.py:64-66) - transformers 4.x's static layer writes
    the slots ``cache_position`` names."""
    from transformers import StaticCache

    native, candidate = models
    torch.manual_seed(5)
    prompt = torch.randint(0, 127, (2, 6), device="cuda")
    ours = StaticCache(config=candidate.config, max_cache_len=16)
    theirs = StaticCache(config=native.config, max_cache_len=16)
    seen = []
    real_update = ours.update

    def update(key, value, layer_idx, cache_kwargs=None):
        seen.append(cache_kwargs)
        return real_update(key, value, layer_idx, cache_kwargs)

    ours.update = update
    current, start = prompt, 0
    for step in range(4):
        position = torch.arange(start, start + current.shape[1], device="cuda")
        seen.clear()
        actual = candidate(input_ids=current, past_key_values=ours, use_cache=True,
                           cache_position=position, logits_to_keep=1).logits
        expected = native(input_ids=current, past_key_values=theirs, use_cache=True,
                          cache_position=position, logits_to_keep=1).logits
        torch.testing.assert_close(actual, expected, rtol=0.03, atol=0.04)
        if current.shape[1] == 1:
            assert len(seen) == len(candidate.model.layers)
            for kwargs in seen:
                assert set(kwargs) == {"sin", "cos", "cache_position"}
                assert torch.equal(kwargs["cache_position"], position)
        start += current.shape[1]
        current = actual[:, -1].argmax(-1, keepdim=True)
