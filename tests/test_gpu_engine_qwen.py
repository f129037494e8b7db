"""The Engine at Qwen3-4B widths on the MI355X, against native transformers.

The benchmark's engine lines time the real architecture (hidden 2560, MLP
9728, 32 query and 8 key/value heads of 128, vocabulary 151,936); this test
runs that architecture with a few layers, so every path those lines time is
composed and checked end to end:

* batch 1: the one-workgroup-per-CU projections with the add + norm folded
  into them, and a 545-token prompt whose cache splits into many key
  segments (the attention's merge launch);
* batch 2: gate/up normalising its input inside the matrix-core tiles, and
  a 2 x 2048 prompt - 4,096 rows, the prefill attention's 8-wave form;
* batch 3: the folded path with three rows padded to four;
* batches 4, 8, 12 and 16: the split-K projections with separate add + norm
  launches;
* every batch: the LM head over the full 151,936-column vocabulary fused
  with the greedy choice, inside the captured decode graph.

Teacher-forced as the contract's judge replays (QWEN_ENGINE_CONTRACT.md:105-123
of the reference; tests/test_qk_norm_rope.py:201-220 and
tests/test_prefill.py:469-497 there): a float32 copy of the same bf16
weights scores prompt + the engine's own tokens on the GPU.  At every step

* each emitted token is within 2.0 logits of the native maximum, and is the
  native argmax wherever the native top two are more than 0.25 apart;
* the engine's bf16 logits are within rtol 0.02 / atol ``ATOL`` of the
  float32 ones (bf16 activations in every layer against a float32 forward),
  and their mean error stays below ``MEAN_ERR``.

``initializer_range`` 0.03 spreads the logits to a standard deviation of
about 1.5 (Qwen3's own 0.02 gives about 1.0 at this width), so the checks
have teeth; the test asserts the spread.
"""

from __future__ import annotations

import copy

import pytest
import torch
from transformers import Qwen3Config

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.engine import Engine  # noqa: E402

QWEN3_4B = dict(vocab_size=151936, hidden_size=2560, intermediate_size=9728,
                num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                max_position_embeddings=40960, rope_theta=5_000_000, rms_norm_eps=1e-6,
                tie_word_embeddings=True, initializer_range=0.03)
LAYERS = 3
#: Measured on the MI355X: max error 0.107-0.141 and mean error 0.0187-0.0193
#: over the five cases (logit standard deviation 1.52).
ATOL = 0.2
MEAN_ERR = 0.025


@pytest.fixture(scope="module")
def engines():
    engine = Engine(config=Qwen3Config(num_hidden_layers=LAYERS, **QWEN3_4B), seed=11,
                    keep_logits=True)
    native = copy.deepcopy(engine.model).float().eval()
    yield engine, native
    del engine, native
    torch.cuda.empty_cache()


def run(engine, prompts, steps):
    tokens, logits = [], []
    for out in engine.generate(prompts, steps):
        assert len(out) == len(prompts) and all(isinstance(t, int) for t in out)
        tokens.append(out)
        logits.append(engine.last_logits.float().clone())
    assert len(tokens) == steps
    return torch.tensor(tokens).T, torch.stack(logits, 1)   # [B, steps] (CPU), [B, steps, V]


@pytest.mark.parametrize("batch,length,steps", [(1, 545, 4), (2, 2048, 3), (3, 600, 3),
                                                (4, 1100, 3), (8, 300, 3), (12, 200, 3),
                                                (16, 641, 3)])
def test_qwen3_4b_widths_teacher_forced(engines, batch, length, steps):
    engine, native = engines
    g = torch.Generator().manual_seed(4000 + 7 * batch + length)
    prompts = torch.randint(0, QWEN3_4B["vocab_size"], (batch, length), generator=g)
    tokens, logits = run(engine, prompts.tolist(), steps)
    state = engine.state
    # the paths this case exists for
    if batch == 1:
        assert state.fold_norms and state.fold_attention and state.attention.splits >= 8
    if batch == 2:
        assert state.fold_norms and state.tiled_gate_up
    if batch == 3:
        assert state.fold_norms
    if batch >= 4:
        assert not state.fold_norms and state.attention.splits >= 2
    full = torch.cat([prompts, tokens[:, :-1]], dim=1).cuda()
    with torch.inference_mode():
        expected = native(input_ids=full, logits_to_keep=steps).logits.float()   # [B, steps, V]
    spread = float(expected.std())
    err = (logits - expected).abs()
    top2 = expected.topk(2, dim=-1)
    chosen = expected.gather(-1, tokens.cuda().unsqueeze(-1)).squeeze(-1)
    gap = top2.values[..., 0] - chosen
    clear = (top2.values[..., 0] - top2.values[..., 1]) > 0.25
    print(f"\nbatch {batch} x {length}: splits {state.attention.splits}, logit std {spread:.3f}, "
          f"max err {float(err.max()):.4f}, mean err {float(err.mean()):.5f}, "
          f"99.99% {float(err.flatten().topk(max(1, err.numel() // 10000)).values[-1]):.4f}, "
          f"max gap {float(gap.max()):.4f}, clear {int(clear.sum())}/{clear.numel()}", flush=True)
    assert spread > 1.2
    assert float(gap.max()) <= 2.0
    assert torch.equal(tokens.cuda()[clear], top2.indices[..., 0][clear])
    assert bool(clear.any())
    torch.testing.assert_close(logits, expected, rtol=0.02, atol=ATOL)
    assert float(err.mean()) < MEAN_ERR
