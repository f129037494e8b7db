"""The Engine harness on the MI355X: every fused kernel of this package inside
one greedy generation loop, against native transformers.

Teacher-forced like the reference's own pipeline test
(tests/test_small_query_attention.py:364-378, tests/test_skinny_gemm.py:323-330):
the native model (float32, CPU, same bf16 weights) scores the prompt plus the
engine's tokens; at every step the engine's logits must be close to the
native ones (rtol 0.02, atol 0.125), its token may trail the native argmax by
at most 2.0 logits, and wherever the native top two differ by more than 0.25
it must be the native argmax.  Graph replay must equal eager stepping bit for bit,
and a local safetensors checkpoint must give the same generation.

A generation abandoned by its consumer, or one whose prefill raised, leaves
the engine usable for the next call.

The contract cases of tests/test_qk_norm_rope.py:201-220 in the reference
((3, 7, 5) twice, (1, 1, 3), (2, 13, 1), (2, 13, 0)): exactly ``count``
lists of ``batch`` ids, each token within 2.0 logits of the native maximum
over the engine's own prefix.  Switching shapes keeps one state, so device
memory does not grow with the number of shapes seen.
"""

from __future__ import annotations

import copy

import pytest
import torch
from transformers import Qwen3Config

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.engine import Engine  # noqa: E402

TINY = dict(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, head_dim=128,
            max_position_embeddings=4096, rope_theta=5_000_000, tie_word_embeddings=True,
            initializer_range=0.1)  # logits spread over ~10, so the checks below have teeth


def run(engine, prompts, steps):
    tokens, logits = [], []
    for out in engine.generate(prompts, steps):
        assert isinstance(out, list) and len(out) == len(prompts) and all(isinstance(t, int) for t in out)
        tokens.append(out)
        logits.append(engine.last_logits.float().cpu().clone())
    assert len(tokens) == steps
    return torch.tensor(tokens).T, torch.stack(logits, 1)  # [B, steps], [B, steps, V]


@pytest.fixture(scope="module")
def engine():
    return Engine(config=Qwen3Config(**TINY), seed=3, keep_logits=True)


@pytest.mark.parametrize("batch,length,steps", [(1, 5, 6), (1, 70, 4), (3, 37, 5), (4, 64, 4)])
def test_generation_matches_native_teacher_forced(engine, batch, length, steps):
    g = torch.Generator().manual_seed(batch * 100 + length)
    prompts = torch.randint(0, TINY["vocab_size"], (batch, length), generator=g).tolist()
    tokens, logits = run(engine, prompts, steps)
    check_teacher_forced(engine, prompts, tokens, logits)
    if (batch, length) == (1, 70):  # two key segments: o_proj merges them itself
        assert engine.state.merged_o


def check_teacher_forced(engine, prompts, tokens, logits):
    length = len(prompts[0])
    native = copy.deepcopy(engine.model).float().cpu()
    full = torch.cat([torch.tensor(prompts), tokens[:, :-1]], dim=1)
    with torch.inference_mode():
        expected = native(input_ids=full).logits[:, length - 1:]   # [B, steps, V]
    assert float(expected.std()) > 1.0
    torch.testing.assert_close(logits, expected, rtol=0.02, atol=0.125)
    chosen = expected.gather(-1, tokens.unsqueeze(-1)).squeeze(-1)
    assert float((expected.amax(-1) - chosen).max()) <= 2.0
    # where the native top two are clearly apart, the engine picks the same token
    top2 = expected.topk(2, dim=-1).values
    clear = (top2[..., 0] - top2[..., 1]) > 0.25
    assert torch.equal(tokens[clear], expected.argmax(-1)[clear])
    assert bool(clear.any())


#: Widths at which the decode step folds the add + norm after the down
#: projection into the down and qkv projections (N = 256 c columns).
ROWS = dict(TINY, hidden_size=512, intermediate_size=1024)


@pytest.mark.parametrize("batch,length", [(1, 21), (2, 21), (3, 21), (4, 21), (1, 300)])
def test_folded_norms_match_native_and_the_split_path(batch, length, monkeypatch):
    """With the fold on (batch <= 3 in the engine; here raised to 4 to cover
    every row count) o_proj and down add the residual and gate/up and the
    next qkv projection normalise their input (no add + norm launches):
    teacher-forced against native like the split-K path, and close to that
    path itself."""
    import starter_amd.engine as engine_module
    monkeypatch.setattr(engine_module, "FOLD_BATCH", 4)  # the engine folds batch <= 3 by default
    cfg = Qwen3Config(**ROWS)
    g = torch.Generator().manual_seed(7 + batch + length)
    prompts = torch.randint(0, ROWS["vocab_size"], (batch, length), generator=g).tolist()
    folded = Engine(config=cfg, seed=5, keep_logits=True)
    tokens, logits = run(folded, prompts, 5)
    assert folded.state.fold_norms and folded.state.fold_attention
    if length == 300:
        assert folded.state.attention.splits > 1
    check_teacher_forced(folded, prompts, tokens, logits)
    split = Engine(config=cfg, seed=5, keep_logits=True, fold_norms=False)
    split_tokens, split_logits = run(split, prompts, 5)
    assert not split.state.fold_norms
    # steps whose prefix agrees see the same inputs: only the projections'
    # accumulation order differs
    same = (tokens == split_tokens).long().cumprod(1)
    agree = torch.cat([torch.ones_like(same[:, :1]), same[:, :-1]], 1).bool()
    assert bool(agree[:, 1:].any())
    torch.testing.assert_close(logits[agree], split_logits[agree], rtol=0.02, atol=0.05)


@pytest.mark.parametrize("batch,length", [(1, 21), (2, 300)])
def test_folded_norms_with_tiled_gate_up(batch, length, monkeypatch):
    """Where the one-workgroup-per-CU SiLU epilogue cannot serve the batch
    (Qwen3-4B at batch 2; forced here) gate/up normalises its input inside
    the matrix-core tiles: teacher-forced against native like the other
    paths."""
    import starter_amd.engine as engine_module
    monkeypatch.setattr(engine_module.row_gemv, "supports_silu_shape", lambda *args: False)
    cfg = Qwen3Config(**ROWS)
    g = torch.Generator().manual_seed(17 + batch + length)
    prompts = torch.randint(0, ROWS["vocab_size"], (batch, length), generator=g).tolist()
    folded = Engine(config=cfg, seed=5, keep_logits=True)
    tokens, logits = run(folded, prompts, 5)
    assert folded.state.fold_attention and folded.state.tiled_gate_up
    check_teacher_forced(folded, prompts, tokens, logits)


def test_default_fold_rule():
    """The engine folds the add + norm launches up to batch 3 (3 rows run
    padded to 4 on the row kernels) and keeps the split-K path from batch 4."""
    eng = Engine(config=Qwen3Config(**ROWS), seed=5)
    for batch, folded in ((1, True), (2, True), (3, True), (4, False)):
        prompt = [[(3 * i + j) % ROWS["vocab_size"] for j in range(9)] for i in range(batch)]
        assert len(list(eng.generate(prompt, 2))) == 2
        assert eng.state.fold_norms == folded, batch


def test_folded_o_proj_merge_variants_agree(monkeypatch):
    """The attention's segments merged inside o_proj (every workgroup) or by
    the attention's own merge launch: the same bits either way."""
    import starter_amd.engine as engine_module
    cfg = Qwen3Config(**ROWS)
    prompts = [list(range(3, 303))]
    merge_in_o_proj = True
    monkeypatch.setattr(engine_module, "MERGE_IN_O_PROJ", merge_in_o_proj)
    eng = Engine(config=cfg, seed=5, keep_logits=True)
    tokens, logits = run(eng, prompts, 4)
    assert eng.state.fold_attention and eng.state.attention.splits > 1
    monkeypatch.setattr(engine_module, "MERGE_IN_O_PROJ", not merge_in_o_proj)
    other = Engine(config=cfg, seed=5, keep_logits=True)
    other_tokens, other_logits = run(other, prompts, 4)
    assert torch.equal(tokens, other_tokens)
    assert torch.equal(logits, other_logits)


def test_graph_replay_equals_eager(engine):
    prompts = [[7, 8, 9, 10, 11, 12, 13], [1, 2, 3, 4, 5, 6, 7]]
    graph_tokens, graph_logits = run(engine, prompts, 5)
    eager = Engine(config=Qwen3Config(**TINY), seed=3, use_graphs=False, keep_logits=True)
    eager_tokens, eager_logits = run(eager, prompts, 5)
    assert torch.equal(graph_tokens, eager_tokens)
    assert torch.equal(graph_logits, eager_logits)
    # a second call of the same shape replays both captured graphs
    graphs = (engine.state.prefill_graph, engine.state.graph)
    assert all(g is not None for g in graphs)
    again_tokens, again_logits = run(engine, prompts, 5)
    assert torch.equal(again_tokens, graph_tokens) and torch.equal(again_logits, graph_logits)
    assert (engine.state.prefill_graph, engine.state.graph) == graphs
    # new prompt content of the same shape: the replayed prefill reads it
    other = [[99, 98, 97, 96, 95, 94, 93], [3, 1, 4, 1, 5, 9, 2]]
    new_tokens, new_logits = run(engine, other, 5)
    eager_tokens, eager_logits = run(eager, other, 5)
    assert torch.equal(new_tokens, eager_tokens) and torch.equal(new_logits, eager_logits)
    assert not torch.equal(new_logits, graph_logits)


def test_abandoned_generation_keeps_a_usable_state(engine):
    """A consumer that stops after two of six steps (the generator closed
    early) leaves the state usable: the next call of the same shape gives the
    uninterrupted result, on the same buffers, which the captured graphs
    address (engine/decode.py keeps its buffer addresses across prompts,
    tests/test_decode.py:91 in the reference)."""
    prompts = [[11, 12, 13, 14, 15], [21, 22, 23, 24, 25]]
    full_tokens, full_logits = run(engine, prompts, 6)
    st = engine.state
    buffers = (st.prompt, st.tokens, st.position, st.used, st.keys[0], st.values[-1])
    addresses = [t.data_ptr() for t in buffers]
    stream = engine.generate(prompts, 6)
    next(stream)
    next(stream)
    stream.close()
    again_tokens, again_logits = run(engine, prompts, 6)
    assert engine.state is st
    assert [t.data_ptr() for t in buffers] == addresses
    assert torch.equal(again_tokens, full_tokens) and torch.equal(again_logits, full_logits)


def test_prefill_error_leaves_the_engine_usable(engine, monkeypatch):
    """An exception raised inside the prefill (here injected into its first
    warm-up run on a new shape) reaches the caller, and the next call of that
    shape captures and generates as if nothing had happened
    (tests/test_prefill.py:447-466 in the reference)."""
    prompts = [[31, 32, 33, 34, 35, 36]]
    real = engine._prefill
    calls = []

    def failing(st):
        calls.append(st.key)
        if len(calls) == 1:
            raise RuntimeError("injected")
        return real(st)

    monkeypatch.setattr(engine, "_prefill", failing)
    with pytest.raises(RuntimeError, match="injected"):
        list(engine.generate(prompts, 4))
    assert torch.cuda.current_stream() == torch.cuda.default_stream()
    tokens, logits = run(engine, prompts, 4)
    monkeypatch.undo()
    fresh = Engine(config=Qwen3Config(**TINY), seed=3, keep_logits=True)
    fresh_tokens, fresh_logits = run(fresh, prompts, 4)
    assert torch.equal(tokens, fresh_tokens) and torch.equal(logits, fresh_logits)


def test_caller_graphs_capture_after_generation():
    """After a generation (whose prefill and decode graphs stay alive), a
    graph the caller captures outside inference mode still captures and
    replays: the engine's captures leave torch's graph RNG state ordinary
    tensors."""
    other = Engine(config=Qwen3Config(**TINY), seed=4)
    assert len(list(other.generate([[1, 2, 3, 4]], 3))) == 3
    assert other.state.graph is not None and not torch.is_inference_mode_enabled()
    x = torch.zeros(4, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y = x + 1
    graph.replay()
    torch.cuda.synchronize()
    assert y.tolist() == [1.0] * 4


def test_local_checkpoint(engine, tmp_path):
    engine.model.save_pretrained(tmp_path, safe_serialization=True)
    loaded = Engine(str(tmp_path), keep_logits=True)
    prompts = [[5, 4, 3, 2, 1, 0, 9, 8]]
    assert torch.equal(run(loaded, prompts, 4)[0], run(engine, prompts, 4)[0])


def _own_prefix_gap(model, prompt, emitted):
    """Largest gap between the native maximum and the emitted token's logit,
    the native model scoring the prompt plus the engine's own tokens."""
    length = len(prompt[0])
    tokens = torch.tensor(emitted).T                          # [B, count]
    own = torch.cat([torch.tensor(prompt), tokens[:, :-1]], dim=1)
    with torch.inference_mode():
        logits = model(input_ids=own).logits[:, length - 1:].float()
    gap = logits.amax(-1) - logits.gather(-1, tokens[..., None]).squeeze(-1)
    assert bool(torch.isfinite(gap).all())
    return float(gap.max())


def test_contract_shapes(engine):
    native = copy.deepcopy(engine.model).float().cpu()
    g = torch.Generator().manual_seed(31)
    for batch, length, count in ((3, 7, 5), (3, 7, 5), (1, 1, 3), (2, 13, 1), (2, 13, 0)):
        prompt = torch.randint(0, TINY["vocab_size"], (batch, length), generator=g).tolist()
        emitted = list(engine.generate(prompt, count))
        assert len(emitted) == count
        if count == 0:
            continue
        assert all(len(row) == batch and all(isinstance(t, int) for t in row) for row in emitted)
        assert _own_prefix_gap(native, prompt, emitted) <= 2.0


def test_one_state_at_a_time():
    """Shapes A, B, A, B: the second visit of a shape holds the same device
    memory as the first (the previous state and its graphs are released)."""
    engine = Engine(config=Qwen3Config(**TINY), seed=5)
    shapes = ((2, 40, 6), (4, 100, 9))
    seen = {}
    for _ in range(2):
        for batch, length, count in shapes:
            prompt = [[(7 * i + j) % TINY["vocab_size"] for j in range(length)] for i in range(batch)]
            assert len(list(engine.generate(prompt, count))) == count
            torch.cuda.synchronize()
            seen.setdefault((batch, length, count), []).append(torch.cuda.memory_allocated())
            assert engine.state.key == (batch, length, count)
    for first, second in seen.values():
        assert second <= first


def test_tuned_gemms_serve_the_prefill_gate_up_shape():
    """Inside ``tuned_gemms`` the recorded hipBLASLt solution serves the
    Qwen3-4B prefill gate/up shape (8,192 rows) - within bf16 GEMM rounding of
    the default choice - and TunableOp's switches are restored after."""
    import torch.nn.functional as F
    from starter_amd import engine as engine_module
    tunable = torch.cuda.tunable
    before = (tunable.is_enabled(), tunable.tuning_is_enabled())
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(8192, 2560, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(19456, 2560, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    want = F.linear(x, w)
    with engine_module.tuned_gemms(True):
        assert tunable.is_enabled() and not tunable.tuning_is_enabled()
        got = F.linear(x, w)
    assert (tunable.is_enabled(), tunable.tuning_is_enabled()) == before
    assert any(r[1].startswith("tn_19456_8192_2560_") for r in tunable.get_results())
    torch.testing.assert_close(got.float(), want.float(), rtol=2e-2, atol=2e-2)
    with engine_module.tuned_gemms(False):
        assert (tunable.is_enabled(), tunable.tuning_is_enabled()) == before
