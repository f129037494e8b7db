"""Engine-shaped greedy generation over the fused HIP kernels.

Same interface as the reference's ``engine/engine.py`` (jadenpxrk/starter,
README.md:49-66): ``Engine(model_path)`` loads a Qwen3 checkpoint and
``generate(input_ids, max_new_tokens)`` yields one ``list[int]`` (a token id
per sequence) per output step, exactly ``max_new_tokens`` times.  Built from
scratch on this package's kernels to show them composing inside the loop the
reference runs:

* prefill (``engine/prefill.py:26-66``): embedding gather, RMSNorm, packed QKV
  projection (hipBLASLt), ``prefill_qkv`` (Q/K norm + RoPE + K/V cache write),
  causal flash attention with grouped K/V heads (``prefill_attention``: one
  launch, no score matrix in memory), and the residual-add + RMSNorm / SiLU *
  up fusions;
  captured once per (batch, prompt length) in a HIP graph and replayed for
  every prompt of that shape (``engine/prefill.py:65-99``);
* decode (``engine/decode_step.py:33-64``): the split-K projections whose f32
  partials feed ``add_rms_norm`` and the split-KV decode attention (which
  also does ``qkv_norm_rope_cache``'s Q/K norm, RoPE and cache write in its
  own launches), the fused gate/up projection with its SiLU epilogue, and
  the LM head fused with the greedy token choice; at batch 1 the
  projections run one workgroup per compute unit over the whole K range,
  so both residual adds move into the epilogues of o_proj and down, and
  both RMSNorms into the prologues of gate/up and the next qkv projection
  (two launches fewer per layer, bit-identical normalised rows; at batch 2
  gate/up normalises its input inside the split-K matrix-core tiles
  instead, whose row kernel cannot serve two rows); the whole step is
  captured once per (batch, capacity) in a HIP graph and replayed with the
  position and cache lengths advanced on the device.

Tokens reach the host as ``engine/decode.py:110-128`` moves them: step k's
device-to-host copy into pinned memory is queued before step k + 1 is
launched, so the GPU runs the next step while the host hands out this one.

Weights come from transformers' ``Qwen3ForCausalLM`` - from a local
checkpoint directory, or randomly initialised from a config - and are packed
once (Q|K|V and gate|up rows, as ``engine/engine.py:39-47`` packs them); the
model's own projection modules are re-pointed at row ranges of the packed
tensors, so no weight is held twice.  One generation state (caches, tables,
graphs) is kept at a time, for the most recent (batch, prompt length, new
tokens), as ``engine/engine.py:62-64`` keeps one.  There is no CPU path: the
engine needs a GPU and the HIP library.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path

import torch
from torch import nn
from torch.nn import functional as F

from .kernels.decode_fused import add_rms_norm, silu_mul
from .kernels.embedding import embedding
from .kernels import lm_head as _lm_head
from .kernels.prefill import prefill_attention, prefill_qkv
from .kernels.rmsnorm import rms_norm
from .kernels.rotary import rope_tables
from .kernels import row_gemv
from .kernels.skinny_gemm import (linear_partials, linear_partials_merged, linear_silu_mul,
                                  linear_silu_mul_normed, supports, supports_merged,
                                  supports_normed_shape)
from .kernels.small_query_attention import SmallQueryAttention

HEAD = 128


@dataclass
class PackedLayer:
    """One decoder layer's weights in the layout the fused path reads."""
    qkv: torch.Tensor        # [(Hq + 2 Hkv) * 128, H]: q rows, k rows, v rows
    o: torch.Tensor          # [H, Hq * 128]
    gate_up: torch.Tensor    # [2 I, H]: gate rows, up rows
    down: torch.Tensor       # [H, I]
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    eps_in: float
    eps_post: float
    eps_q: float
    eps_k: float


@torch.no_grad()
def _pack_rows(*modules) -> torch.Tensor:
    """Concatenate the modules' weights along the output rows and make each
    module's weight the matching row range of the result (one copy in memory,
    as engine/qk_norm_rope.py:22-30 does for Q|K|V)."""
    packed = torch.cat([m.weight for m in modules]).contiguous()
    start = 0
    for module in modules:
        stop = start + module.weight.shape[0]
        module.weight = nn.Parameter(packed[start:stop], requires_grad=False)
        start = stop
    return packed


def pack_layer(layer) -> PackedLayer:
    """Pack a transformers ``Qwen3DecoderLayer`` (any device / dtype kept); its
    q/k/v and gate/up modules then read the packed storage."""
    attn, mlp = layer.self_attn, layer.mlp
    return PackedLayer(
        qkv=_pack_rows(attn.q_proj, attn.k_proj, attn.v_proj),
        o=attn.o_proj.weight.contiguous(),
        gate_up=_pack_rows(mlp.gate_proj, mlp.up_proj),
        down=mlp.down_proj.weight.contiguous(),
        ln_in=layer.input_layernorm.weight.contiguous(),
        ln_post=layer.post_attention_layernorm.weight.contiguous(),
        q_norm=attn.q_norm.weight.contiguous(),
        k_norm=attn.k_norm.weight.contiguous(),
        eps_in=float(layer.input_layernorm.variance_epsilon),
        eps_post=float(layer.post_attention_layernorm.variance_epsilon),
        eps_q=float(attn.q_norm.variance_epsilon),
        eps_k=float(attn.k_norm.variance_epsilon),
    )


def check_rotary(model) -> None:
    """The rotary tables are built from ``inv_freq`` alone (the default RoPE);
    refuse checkpoints whose rotary module scales or reshapes the angles."""
    rope = model.model.rotary_emb
    kind = getattr(rope, "rope_type", "default")
    scaling = float(getattr(rope, "attention_scaling", 1.0))
    if kind != "default" or scaling != 1.0:
        raise ValueError(f"the engine implements the default RoPE only, not rope_type {kind!r} "
                         f"with attention_scaling {scaling}")


#: Largest batch whose decode step merges attention segments inside o_proj
#: (split-K path; every column tile re-merges its heads' segments, so larger
#: batches lose: 2,806 against 2,389 us/step at 4 x 2048, 3,364 against 2,480
#: at 8 x 1024, 4,468 against 2,669 at 16 x 512, same tokens).
MERGED_O_BATCH = 1
#: Key-segment granularity of the decode attention's plan: the segment count
#: of partition_keys with lengths balanced to 16 keys (4 x 2081 keys: 8 x 272
#: instead of 7 x 320, 10.6 against 11.3 us; 16 x 641: 2 x 336 instead of
#: 2 x 384, 11.8 against 12.2 us; batch 1 unchanged).
KEY_ALIGN = 16

#: Largest batch whose decode step folds the add + norm launches into the
#: projections around them where their shapes allow (measured on Qwen3-4B:
#: batch 1 1,989 against 2,121 us/step with the down/qkv fold alone and
#: ~2,190 with neither; batch 2 with both folds - gate/up on the normalising
#: matrix-core tiles - 2,092-2,096 against 2,135-2,139 with the down/qkv fold
#: alone and 2,194-2,196 with neither at 512 prompt tokens, 2,168-2,170
#: against 2,214-2,221 at 2,048.  With the normalising prologues waiting for
#: the sums of squares only: batch 3 2,136-2,187 against 2,213-2,216 at 512
#: prompt tokens, 2,249-2,294 against 2,324-2,326 at 2,048; batch 4
#: 2,251-2,263 against 2,258-2,262 at 512 and 2,392-2,394 against
#: 2,392-2,394 at 2,048: no gain there).
FOLD_BATCH = 3
#: Whether the folded path merges the attention's segments inside o_proj
#: (every workgroup merges every head: 2,154 us/step at batch 1) instead of
#: taking the attention's own merge launch (1,989 us/step).
MERGE_IN_O_PROJ = False
#: hipBLASLt solutions for the prefill projections where one measured faster
#: than the library's default choice on MI355X (torch TunableOp's results
#: format, read with tuning switched off; torch checks the file's torch, HIP,
#: hipBLASLt and GPU versions and ignores it when they differ).  One entry:
#: the Qwen3-4B gate/up projection at 8,192 prompt rows, 586 against 667 us
#: with the weights streamed from HBM; the other projections at 512, 2,048
#: and 8,192 rows gained nothing.
TUNED_GEMMS = Path(__file__).with_name("tuned_gemms_gfx950.csv")
_tuned_gemms_loaded: bool | None = None


@contextmanager
def tuned_gemms(active: bool = True):
    """Within the block, torch's projections take the recorded solutions of
    ``TUNED_GEMMS`` (TunableOp on, tuning off; every other shape keeps the
    default choice); TunableOp's previous switches are restored after.  A
    HIP graph captured inside keeps the chosen kernels for its replays."""
    global _tuned_gemms_loaded
    tunable = torch.cuda.tunable
    if active and _tuned_gemms_loaded is None:
        try:
            _tuned_gemms_loaded = TUNED_GEMMS.exists() and bool(tunable.read_file(str(TUNED_GEMMS)))
        except RuntimeError:  # a torch build without TunableOp, or a table it cannot parse
            _tuned_gemms_loaded = False
    if not (active and _tuned_gemms_loaded):
        yield
        return
    previous = (tunable.is_enabled(), tunable.tuning_is_enabled())
    tunable.tuning_enable(False)
    tunable.enable(True)
    try:
        yield
    finally:
        tunable.enable(previous[0])
        tunable.tuning_enable(previous[1])


#: Whether the folded path's gate/up projection may run as the matrix-core
#: tiles with the RMSNorm in their prologue (``skinny_gemm.linear_silu_mul_normed``)
#: where the one-workgroup-per-CU kernel's SiLU epilogue cannot serve the
#: batch (2 rows x 76 columns per workgroup).  At batch 1 the row kernel
#: stays (18.7 us against 18.9 for the tiles on Qwen3-4B, whose plain form
#: takes 16.9: every workgroup's prologue reads the same sums of squares,
#: row and gain at once), and so does qkv (7.7 against 10.3 us).
NORMED_TILES = True


class _State:
    """Caches, rotary tables, graphs and host buffers for one (batch, prompt
    length, new tokens)."""

    def __init__(self, engine: "Engine", batch: int, length: int, new_tokens: int):
        dev = engine.device
        capacity = length + new_tokens
        self.key = (batch, length, new_tokens)
        self.batch, self.length, self.capacity = batch, length, capacity
        shape = (batch, engine.kv_heads, capacity, HEAD)
        self.keys = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in engine.layers]
        self.values = [torch.zeros(shape, dtype=torch.bfloat16, device=dev) for _ in engine.layers]
        self.cos, self.sin = rope_tables(engine.inv_freq, capacity, device=dev)
        self.attention = SmallQueryAttention(batch, engine.q_heads, engine.kv_heads, capacity, dev,
                                             key_align=KEY_ALIGN)
        # o_proj merges the attention's key segments itself (one launch fewer
        # per layer) up to MERGED_O_BATCH sequences.
        self.merged_o = (batch <= MERGED_O_BATCH and self.attention.splits > 1
                         and supports_merged(self.attention.partials, self.attention.stats, batch,
                                             engine.layers[0].o))
        # Down projection with the residual add, next qkv projection with the
        # RMSNorm (no add + norm launch between them) where the shapes allow.
        first = engine.layers[0]
        self.fold_norms = (engine.fold_norms and batch <= FOLD_BATCH and len(engine.layers) > 1
                           and row_gemv.supports_shape(batch, first.down.shape[1],
                                                       first.down.shape[0])
                           and row_gemv.supports_shape(batch, first.qkv.shape[1],
                                                       first.qkv.shape[0]))
        # o_proj with the residual add (merging the attention's segments),
        # gate/up with the RMSNorm: the add + norm after the attention.
        hidden, inner = first.o.shape[0], first.down.shape[1]
        splits = self.attention.splits
        o_ok = (row_gemv.supports_merged_shape(batch, splits, engine.q_heads, engine.kv_heads,
                                               hidden) if MERGE_IN_O_PROJ and splits > 1 else
                row_gemv.supports_shape(batch, first.o.shape[1], hidden))
        row_silu = row_gemv.supports_silu_shape(batch, hidden, inner)
        self.tiled_gate_up = (NORMED_TILES and not row_silu
                              and supports_normed_shape(batch, hidden, inner, pairs=True))
        self.fold_attention = (engine.fold_norms and batch <= FOLD_BATCH and o_ok
                               and (row_silu or self.tiled_gate_up))
        self.prompt = torch.zeros((batch, length), dtype=torch.int64, device=dev)
        self.tokens = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.position = torch.zeros(1, dtype=torch.int64, device=dev)
        self.used = torch.zeros(batch * engine.kv_heads, dtype=torch.int32, device=dev)
        # the step whose tokens the host reads, copied into pinned memory
        self.host = torch.empty(batch, dtype=torch.int64, pin_memory=True)
        self.ready = torch.cuda.Event()
        # graphs need the fused LM head (torch's argmax records a memset node)
        self.graphable = engine.use_graphs and batch <= _lm_head.MAX_ROWS
        self.prefill_graph = None
        self.prefill_logits = None
        self.graph = None
        self.logits = None


class Engine:
    """Greedy Qwen3 generation on the fused gfx950 kernels (see module doc)."""

    def __init__(self, model_path: str | None = None, *, config=None, seed: int = 0,
                 device: str | torch.device = "cuda", use_graphs: bool = True,
                 keep_logits: bool = False, fold_norms: bool = True, tuned_gemms: bool = True):
        """``keep_logits``: also keep each step's bf16 logits in ``last_logits``
        (a device copy per step; for tests and inspection).  ``fold_norms``:
        up to FOLD_BATCH sequences fold the add + norm launches of a layer
        into the projections around them where the shapes allow (off: the
        split-K path at every batch).  ``tuned_gemms``: the prefill's
        projections take the recorded hipBLASLt solutions of TUNED_GEMMS
        where one exists for their shape."""
        from transformers import Qwen3ForCausalLM
        self.device = torch.device(device)
        if self.device.type != "cuda" or not torch.cuda.is_available():
            raise RuntimeError("Engine needs a GPU: the fused kernels have no CPU path")
        if model_path is not None:
            model = Qwen3ForCausalLM.from_pretrained(model_path, torch_dtype=torch.bfloat16,
                                                     local_files_only=True)
        elif config is not None:
            torch.manual_seed(seed)
            with torch.device(self.device):  # initialise on the GPU (seconds for 4B params)
                model = Qwen3ForCausalLM(config).to(torch.bfloat16)
        else:
            raise ValueError("give a local checkpoint directory or a Qwen3Config")
        model = model.to(self.device).eval()
        check_rotary(model)
        cfg = model.config
        self.config = cfg
        self.model = model
        self.q_heads, self.kv_heads = cfg.num_attention_heads, cfg.num_key_value_heads
        width = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        if width != HEAD:
            raise ValueError(f"the fused Q/K kernels need head_dim {HEAD}, not {width}")
        self.scale = model.model.layers[0].self_attn.scaling
        with torch.no_grad():
            self.layers = [pack_layer(layer) for layer in model.model.layers]
        self.embed = model.model.embed_tokens.weight
        self.final_norm = model.model.norm.weight
        self.final_eps = float(model.model.norm.variance_epsilon)
        self.lm_head = model.lm_head.weight
        self.inv_freq = model.model.rotary_emb.inv_freq.float()
        self.use_graphs = use_graphs
        self.keep_logits = keep_logits
        self.fold_norms = fold_norms
        self.tuned_gemms = tuned_gemms
        self.state: _State | None = None
        self.last_logits = None
        # One side stream for every warm-up and capture: torch keeps a BLAS
        # workspace per stream it has run a projection on, for the life of
        # the process, so a fresh stream per capture would leak one each.
        self._capture_stream = torch.cuda.Stream(self.device)

    # ------------------------------------------------------------ helpers

    @staticmethod
    def _project(x, weight):
        """x @ weight.T as f32 split-K partials when decode-sized, else bf16."""
        return linear_partials(x, weight) if supports(x, weight) else F.linear(x, weight)

    @staticmethod
    def _mlp_hidden(normed, gate_up):
        if supports(normed, gate_up, pairs=True):
            return linear_silu_mul(normed, gate_up)
        return silu_mul(F.linear(normed, gate_up))

    def _select(self, normed, tokens, advance=None):
        """LM head + greedy choice: writes the tokens; returns the bf16 logits
        when ``keep_logits`` (else None) and whether the fused LM head also
        advanced ``advance`` = (position, lengths) by one (the step's last
        writes, without two more launches)."""
        if _lm_head.supports(normed, self.lm_head):
            out = _lm_head.lm_head_argmax(normed, self.lm_head, logits=self.keep_logits,
                                          tokens=tokens, advance=advance)
            return (out[1] if self.keep_logits else None), advance is not None
        logits = F.linear(normed, self.lm_head)
        tokens.copy_(logits.argmax(-1))
        return logits, False

    def _next_norm(self, index):
        if index + 1 < len(self.layers):
            nxt = self.layers[index + 1]
            return nxt.ln_in, nxt.eps_in
        return self.final_norm, self.final_eps

    def _state(self, batch, length, new_tokens) -> _State:
        """The state for this shape; a different shape drops the old state
        (caches, graphs and their memory pools) before allocating the new."""
        key = (batch, length, new_tokens)
        if self.state is None or self.state.key != key:
            self.state = None
            self.last_logits = None
            self.state = _State(self, batch, length, new_tokens)
        return self.state

    # ------------------------------------------------------------ prefill

    def _prefill_attention(self, q, keys, values, length):
        """Causal GQA attention over the prompt, q [B, T, Hq, 128] against the
        first T cache slots (one flash-attention launch: no score matrix in
        memory).  Returns [B * T, Hq * 128]."""
        out = prefill_attention(q, keys, values, length, self.scale)
        return out.view(q.shape[0] * length, self.q_heads * HEAD)

    def _prefill(self, st: _State):
        """Prompt ``st.prompt`` -> K/V cache slots [0, T) of every layer and the
        first token of each sequence in ``st.tokens`` (capturable)."""
        batch, length = st.batch, st.length
        x = embedding(st.prompt.view(-1), self.embed)
        first = self.layers[0]
        normed = rms_norm(x, first.ln_in, first.eps_in)
        last = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            q = prefill_qkv(F.linear(normed, layer.qkv), layer.q_norm, layer.k_norm, layer.eps_q,
                            layer.eps_k, st.cos, st.sin, st.keys[index], st.values[index], length)
            attended = self._prefill_attention(q, st.keys[index], st.values[index], length)
            x, normed = add_rms_norm(x, F.linear(attended, layer.o), layer.ln_post, layer.eps_post)
            hidden = silu_mul(F.linear(normed, layer.gate_up))
            weight, eps = self._next_norm(index)
            if index == last:
                # only each sequence's last position feeds the LM head
                x = x.view(batch, length, -1)[:, -1].contiguous()
                hidden = hidden.view(batch, length, -1)[:, -1].contiguous()
            x, normed = add_rms_norm(x, F.linear(hidden, layer.down), weight, eps)
        return self._select(normed, st.tokens)[0]

    def _run_prefill(self, st: _State):
        """Prefill from a HIP graph captured on the first prompt of this shape
        (warm-up runs first, then capture, then the replay that produces the
        result), as engine/prefill.py:79-99 does; eager when graphs are off."""
        if not st.graphable:
            with tuned_gemms(self.tuned_gemms):
                return self._prefill(st)
        if st.prefill_graph is None:
            current = torch.cuda.current_stream(self.device)
            stream = self._capture_stream
            stream.wait_stream(current)
            with tuned_gemms(self.tuned_gemms):
                with torch.cuda.stream(stream):
                    for _ in range(2):
                        self._prefill(st)
                current.wait_stream(stream)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    st.prefill_logits = self._prefill(st)
            current.wait_stream(stream)
            st.prefill_graph = graph
        st.prefill_graph.replay()
        return st.prefill_logits

    # ------------------------------------------------------------- decode

    def _decode_step(self, st: _State):
        """One token per sequence at slot ``st.position``; advances the
        position and lengths on the device (capturable)."""
        batch = st.batch
        x = embedding(st.tokens, self.embed)
        first = self.layers[0]
        normed = rms_norm(x, first.ln_in, first.eps_in)
        sq = None  # set while x's RMSNorm is left to the next qkv projection
        last = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            if sq is None:
                qkv = self._project(normed, layer.qkv)
            else:
                qkv = row_gemv.linear_normed(x, sq, layer.ln_in, layer.eps_in, layer.qkv)
            # qkv_norm_rope_cache + attention, fused into the attention launches
            args = (qkv, layer.q_norm, layer.k_norm, layer.eps_q,
                    layer.eps_k, st.cos, st.sin, st.position, st.keys[index], st.values[index],
                    st.used, self.scale)
            if st.fold_attention:
                if MERGE_IN_O_PROJ and st.attention.splits > 1:
                    st.attention.run_qkv_unmerged(*args)
                    x, sq = row_gemv.linear_residual_merged(st.attention.partials,
                                                            st.attention.stats, batch, layer.o, x)
                else:
                    attended = st.attention.run_qkv(*args).view(batch, -1)
                    x, sq = row_gemv.linear_residual(attended, layer.o, x)
                normed_mlp = (linear_silu_mul_normed if st.tiled_gate_up
                              else row_gemv.linear_silu_mul_normed)
                hidden = normed_mlp(x, sq, layer.ln_post, layer.eps_post, layer.gate_up)
            else:
                if st.merged_o:
                    st.attention.run_qkv_unmerged(*args)
                    o = linear_partials_merged(st.attention.partials, st.attention.stats, batch,
                                               layer.o)
                else:
                    o = self._project(st.attention.run_qkv(*args).view(batch, -1), layer.o)
                x, normed = add_rms_norm(x, o, layer.ln_post, layer.eps_post)
                hidden = self._mlp_hidden(normed, layer.gate_up)
            if st.fold_norms and index < last:
                x, sq = row_gemv.linear_residual(hidden, layer.down, x)
            else:
                weight, eps = self._next_norm(index)
                x, normed = add_rms_norm(x, self._project(hidden, layer.down), weight, eps)
                sq = None
        logits, advanced = self._select(normed, st.tokens, (st.position, st.used))
        if not advanced:
            st.position.add_(1)
            st.used.add_(1)
        return logits

    def _capture(self, st: _State):
        """Capture the decode step into a HIP graph.  The warm-up runs repeat
        the first step (same token, same slot), so they leave the caches as
        the first replay does; the buffers are restored before replaying."""
        saved = (st.tokens.clone(), st.position.clone(), st.used.clone())
        stream = self._capture_stream
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            for _ in range(2):
                st.tokens.copy_(saved[0]); st.position.copy_(saved[1]); st.used.copy_(saved[2])
                self._decode_step(st)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        st.tokens.copy_(saved[0]); st.position.copy_(saved[1]); st.used.copy_(saved[2])
        with torch.cuda.graph(graph, stream=stream):
            st.logits = self._decode_step(st)
        st.tokens.copy_(saved[0]); st.position.copy_(saved[1]); st.used.copy_(saved[2])
        st.graph = graph

    # ------------------------------------------------------------ generate

    @torch.no_grad()
    def generate(self, input_ids: list[list[int]], max_new_tokens: int):
        """Greedy continuation; yields one list[int] per step, max_new_tokens times.

        Runs under ``no_grad`` rather than ``inference_mode``: the first HIP
        graph captured in a process creates torch's graph-safe RNG state
        tensors, and captured under inference mode they would be inference
        tensors, which every later capture outside inference mode (the
        caller's own graphs) must update in place and cannot while this
        engine's graphs exist."""
        if max_new_tokens <= 0:
            return
        if not input_ids:
            raise ValueError("need at least one sequence")
        length = len(input_ids[0])
        if length < 1 or any(len(row) != length for row in input_ids):
            raise ValueError("every sequence in input_ids must have the same non-zero length")
        batch = len(input_ids)
        st = self._state(batch, length, max_new_tokens)
        st.prompt.copy_(torch.tensor(input_ids, dtype=torch.int64))
        logits = self._run_prefill(st)
        st.position.fill_(length)
        st.used.fill_(length + 1)
        if max_new_tokens > 1 and st.graphable and st.graph is None:
            self._capture(st)
        for step in range(max_new_tokens):
            # queue this step's tokens for the host, then the next step
            st.host.copy_(st.tokens, non_blocking=True)
            if self.keep_logits:
                self.last_logits = logits.clone()
            st.ready.record()
            if step + 1 < max_new_tokens:
                if st.graph is not None:
                    st.graph.replay()
                    logits = st.logits
                else:
                    logits = self._decode_step(st)
            st.ready.synchronize()
            yield st.host.tolist()
