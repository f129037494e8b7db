"""LM head + greedy token choice on the MI355X against the oracle.

Integer-valued inputs give exact logits with many exactly tied maxima: the
logits and the tokens (lowest index among the maxima) must equal the oracle
bit for bit at every dispatch path.  Random inputs: logits >= 99.9% equal to
the exactly rounded ones and elsewhere within f32 accumulation error
(2^-16 sum|x*w|) plus one bf16 rounding of them, the token always the
first maximum of the kernel's own logits, and equal to the oracle's wherever
the oracle's top two logits differ.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import O, assert_bf16_close, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels.lm_head import lm_head_argmax  # noqa: E402

DEV = "cuda"


@pytest.mark.parametrize("m", [1, 3, 4, 5, 8, 9, 16, 17, 33, 64])
# 4112: 16-column tiles only; 4128: a partly filled last 64- or 128-column workgroup
@pytest.mark.parametrize("vocab", [4096, 4112, 4128])
def test_integer_logits_and_tied_tokens_exact(m, vocab):
    g = gen(600 + m + vocab)
    x = torch.zeros(m, 256, dtype=torch.bfloat16)
    x[:, 0] = 1
    x[:, 1:4] = torch.randint(0, 2, (m, 3), generator=g).to(torch.bfloat16)
    w = torch.randint(-1, 2, (vocab, 256), generator=g).to(torch.bfloat16)
    tokens, logits = lm_head_argmax(x.to(DEV), w.to(DEV), logits=True)
    ref_tokens, ref_logits = O.lm_head_argmax(bits(x), bits(w))
    assert_bits_exact(logits, ref_logits, what="logits")
    np.testing.assert_array_equal(tokens.cpu().numpy(), ref_tokens)
    assert torch.equal(tokens, logits.argmax(-1))


@pytest.mark.parametrize("m", [1, 4])
def test_qwen_vocab_random(m):
    g = gen(620 + m)
    x = normal((m, 2560), g=g)
    w = normal((151936, 2560), 0.0, 0.02, g)
    xd, wd = x.to(DEV), w.to(DEV)
    tokens, logits = lm_head_argmax(xd, wd, logits=True)
    ref_tokens, ref_logits = O.lm_head_argmax(bits(x), bits(w))
    # >= 99.9% bit-exact; elsewhere within f32 accumulation error of the exact
    # logit plus one bf16 rounding (near-zero logits cancel, so ulps mislead)
    assert_bf16_close(logits, ref_logits, max_ulp=1 << 16, min_exact=0.999, what="lm head logits")
    got, exp = logits.float().cpu(), torch.from_numpy(O.bf16_value(ref_logits))
    scale = (x.double().abs() @ w.double().abs().T).float()
    assert bool(((got - exp).abs() <= 2.0**-16 * scale + 2.0**-7 * exp.abs()).all())
    assert torch.equal(tokens, logits.argmax(-1))               # the kernel's own first maximum
    ref = torch.from_numpy(O.bf16_value(ref_logits))
    top2 = ref.topk(2, dim=-1).values
    clear = top2[:, 0] > top2[:, 1]
    assert torch.equal(tokens.cpu()[clear], torch.from_numpy(ref_tokens)[clear])
    assert torch.equal(lm_head_argmax(xd, wd), tokens)           # without the logits copy


def test_qwen_vocab_integer_batch64():
    g = gen(640)
    x = torch.zeros(64, 2560, dtype=torch.bfloat16)
    x[:, :3] = torch.randint(0, 2, (64, 3), generator=g).to(torch.bfloat16)
    w = torch.randint(-2, 3, (151936, 2560), generator=g).to(torch.bfloat16)
    tokens = lm_head_argmax(x.to(DEV), w.to(DEV))
    exact = x[:, :3].double() @ w[:, :3].double().T
    np.testing.assert_array_equal(tokens.cpu().numpy(), np.argmax(exact.numpy(), axis=1))


def test_graph_replay_follows_fresh_inputs():
    g = gen(650)
    w = normal((8192, 512), 0.0, 0.05, g).to(DEV)
    x = normal((4, 512), g=g).to(DEV)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            lm_head_argmax(x, w)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        tokens, logits = lm_head_argmax(x, w, logits=True)
    for seed in range(3):
        x.copy_(normal((4, 512), g=gen(660 + seed)).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        eager_tokens, eager_logits = lm_head_argmax(x, w, logits=True)
        assert torch.equal(tokens, eager_tokens) and torch.equal(logits, eager_logits)
        assert torch.equal(tokens, logits.argmax(-1))


def test_advance_entry_matches_and_advances():
    """qf_lm_head_argmax_advance: the same tokens and logits as the plain
    entry, and the position and every length one higher afterwards (the
    decode step's state advance in the same launches), also in a replayed
    graph."""
    g = torch.Generator(device="cuda").manual_seed(91)
    x = torch.randn(3, 512, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(4096, 512, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    want_tokens, want_logits = lm_head_argmax(x, w, logits=True)
    position = torch.tensor([41], dtype=torch.int64, device="cuda")
    lengths = torch.arange(24, dtype=torch.int32, device="cuda") * 7
    start_len = lengths.clone()
    tokens, logits = lm_head_argmax(x, w, logits=True, advance=(position, lengths))
    torch.cuda.synchronize()
    assert torch.equal(tokens, want_tokens) and torch.equal(logits, want_logits)
    assert position.item() == 42 and torch.equal(lengths, start_len + 1)
    out = torch.empty(3, dtype=torch.int64, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        lm_head_argmax(x, w, tokens=out, advance=(position, lengths))
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        lm_head_argmax(x, w, tokens=out, advance=(position, lengths))
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want_tokens)
    assert position.item() == 46 and torch.equal(lengths, start_len + 5)
    with pytest.raises(ValueError):
        lm_head_argmax(x, w, advance=(position.to(torch.int32), lengths))
