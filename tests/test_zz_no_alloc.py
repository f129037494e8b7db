"""The allocation-free LM head entry point (``qf_lm_head_argmax_static``) on
the MI355X, called through the C ABI: its tokens and logits equal those of
``qf_lm_head_argmax`` (same kernels, caller-owned candidates) bit for bit, on
two calls in a row, the second with a smaller input, so nothing the first
call left in the shared static scratch reaches the second result.  Integer
inputs with many exactly tied maxima also pin both against the oracle.
Inputs beyond the scratch capacity are refused on the host.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import O, assert_bits_exact, bits, gen, normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd.kernels import _lib  # noqa: E402

DEV = "cuda"
QF_E_CAPACITY = -4


def run_both(x, w):
    """(tokens, logits) from the workspace entry point and from the static one."""
    lib = _lib.lib()
    rows, k = x.shape
    vocab = w.shape[0]
    stream = _lib.stream(x.device)
    cand = torch.empty((rows, lib.qf_lm_head_blocks(vocab), 2), dtype=torch.int32, device=DEV)
    out = []
    for static in (False, True):
        tokens = torch.full((rows,), -7, dtype=torch.int64, device=DEV)
        logits = torch.full((rows, vocab), float("nan"), dtype=torch.bfloat16, device=DEV)
        if static:
            st = lib.qf_lm_head_argmax_static(x.data_ptr(), rows, k, w.data_ptr(), vocab,
                                              tokens.data_ptr(), logits.data_ptr(), stream)
        else:
            st = lib.qf_lm_head_argmax(x.data_ptr(), rows, k, w.data_ptr(), vocab,
                                       cand.data_ptr(), tokens.data_ptr(), logits.data_ptr(),
                                       stream)
        assert st == 0, lib.qf_error_string(st)
        torch.cuda.synchronize()
        out.append((tokens.cpu(), logits))
    return out


def test_static_scratch_matches_workspace_entry_point():
    g = gen(901)
    # first call: 64 rows over the Qwen3-4B vocabulary (607,744 of the
    # 1,048,576 slots); second: 3 rows of a smaller vocabulary and width
    cases = [(normal((64, 2560), g=g), normal((151936, 2560), 0.0, 0.02, g)),
             (normal((3, 1024), g=g), normal((32000, 1024), 0.0, 0.02, g))]
    for x, w in cases:
        (ref_tokens, ref_logits), (tokens, logits) = run_both(x.to(DEV), w.to(DEV))
        assert torch.equal(tokens, ref_tokens)
        assert_bits_exact(logits, ref_logits, what="logits")
        assert torch.equal(tokens, logits.float().cpu().argmax(-1))
        del ref_logits, logits
    torch.cuda.empty_cache()


def test_static_scratch_exact_ties_against_oracle():
    """Integer inputs: exact logits full of tied maxima.  Big call first, then
    a smaller one whose first slots the big call had filled."""
    g = gen(902)
    for m, vocab in ((40, 8192), (5, 4112)):
        x = torch.zeros(m, 256, dtype=torch.bfloat16)
        x[:, 0] = 1
        x[:, 1:4] = torch.randint(0, 2, (m, 3), generator=g).to(torch.bfloat16)
        w = torch.randint(-1, 2, (vocab, 256), generator=g).to(torch.bfloat16)
        (ref_tokens, ref_logits), (tokens, logits) = run_both(x.to(DEV), w.to(DEV))
        want_tokens, want_logits = O.lm_head_argmax(bits(x), bits(w))
        assert_bits_exact(logits, want_logits, what="static logits")
        np.testing.assert_array_equal(tokens.numpy(), want_tokens)
        assert torch.equal(tokens, ref_tokens)


def test_capacity_refused_before_launch():
    lib = _lib.lib()
    x = torch.zeros((64, 256), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((16 * 16385, 256), dtype=torch.bfloat16, device=DEV)
    tokens = torch.full((64,), -7, dtype=torch.int64, device=DEV)
    st = lib.qf_lm_head_argmax_static(x.data_ptr(), 64, 256, w.data_ptr(), w.shape[0],
                                      tokens.data_ptr(), None, _lib.stream(x.device))
    assert st == QF_E_CAPACITY
    assert b"static scratch" in lib.qf_error_string(st)
    torch.cuda.synchronize()
    assert bool((tokens == -7).all())


def _graph_replays_match(x, w, replays=3):
    """Capture qf_lm_head_argmax_static in a HIP graph (torch.cuda.graph), then
    replay it several times with eager work and synchronisations between the
    replays, each replay against qf_lm_head_argmax run eagerly."""
    lib = _lib.lib()
    rows, k = x.shape
    vocab = w.shape[0]
    tokens = torch.full((rows,), -7, dtype=torch.int64, device=DEV)
    logits = torch.full((rows, vocab), float("nan"), dtype=torch.bfloat16, device=DEV)
    graph = torch.cuda.graph_pool_handle()
    g = torch.cuda.CUDAGraph()
    status = []
    with torch.cuda.graph(g, pool=graph):
        status.append(lib.qf_lm_head_argmax_static(
            x.data_ptr(), rows, k, w.data_ptr(), vocab, tokens.data_ptr(), logits.data_ptr(),
            _lib.stream(x.device)))
    assert status == [0], lib.qf_error_string(status[0])
    cand = torch.empty((rows, lib.qf_lm_head_blocks(vocab), 2), dtype=torch.int32, device=DEV)
    for replay in range(replays):
        x.mul_(-1 if replay % 2 else 1)          # eager work between replays
        tokens.fill_(-7)
        logits.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        want_tokens = torch.empty_like(tokens)
        want_logits = torch.empty_like(logits)
        st = lib.qf_lm_head_argmax(x.data_ptr(), rows, k, w.data_ptr(), vocab, cand.data_ptr(),
                                   want_tokens.data_ptr(), want_logits.data_ptr(),
                                   _lib.stream(x.device))
        assert st == 0, lib.qf_error_string(st)
        torch.cuda.synchronize()
        assert torch.equal(tokens, want_tokens), replay
        assert_bits_exact(logits, want_logits, what=f"replay {replay}")


def test_static_entry_replays_in_a_graph():
    g = gen(903)
    _graph_replays_match(normal((4, 2560), g=g).to(DEV), normal((32768, 2560), 0.0, 0.02, g).to(DEV))


_FIRST_CALL_CAPTURED = r"""
import sys, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
import test_zz_no_alloc as t
from conftest import gen, normal
g = gen(904)
x = normal((2, 1024), g=g).to("cuda")
w = normal((8192, 1024), 0.0, 0.02, g).to("cuda")
# the library's kernels are loaded by an eager call of another entry point;
# the static entry's first call - its address lookup - happens under capture
lib = t._lib.lib()
cand = torch.empty((2, lib.qf_lm_head_blocks(8192), 2), dtype=torch.int32, device="cuda")
tok = torch.empty(2, dtype=torch.int64, device="cuda")
assert lib.qf_lm_head_argmax(x.data_ptr(), 2, 1024, w.data_ptr(), 8192, cand.data_ptr(),
                             tok.data_ptr(), None, t._lib.stream(x.device)) == 0
torch.cuda.synchronize()
t._graph_replays_match(x, w)
print("first-call-under-capture ok", flush=True)
"""


def test_static_entry_first_call_under_capture():
    """In a fresh process the first call of the static entry on the device -
    the one that looks the scratch address up - is made under capture."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    out = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, str(root)],
                         capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-4000:]
    assert "first-call-under-capture ok" in out.stdout
