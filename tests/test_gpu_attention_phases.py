"""The instrumented decode attention (``libqwen_fused_phases.so``, built with
``-DQF_PHASE_STAMPS`` for ``starter_amd.attention_phases``) on the MI355X:
its outputs and cache writes equal the product entry point's bit for bit,
and every workgroup's stamps are ordered."""

from __future__ import annotations

import pytest
import torch

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]

from starter_amd import attention_phases as ph  # noqa: E402
from starter_amd.kernels import _lib  # noqa: E402
from starter_amd.kernels.rotary import default_inv_freq, rope_tables  # noqa: E402
from starter_amd.kernels.small_query_attention import SmallQueryAttention  # noqa: E402


@pytest.mark.parametrize("batch,keys,qkv_splits", [(1, 300, 0), (3, 130, 5), (2, 64, 0)])
def test_stamped_attention_equals_product(batch, keys, qkv_splits):
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(batch + keys)
    nq, nk, d = ph.NQ, ph.NK, ph.D
    width = (nq + 2 * nk) * d
    plan = SmallQueryAttention(batch, nq, nk, keys, dev)
    caches = [torch.randn((batch, nk, keys, d), generator=g, device=dev).to(torch.bfloat16)
              for _ in range(2)]
    qkv = (torch.randn((batch, width), generator=g, device=dev).to(torch.bfloat16) if not qkv_splits
           else torch.randn((qkv_splits, batch, width), generator=g, device=dev))
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(torch.bfloat16)
    cos, sin = rope_tables(default_inv_freq(5e6, d).to(dev), keys, device=dev)
    position = torch.full((1,), keys - 1, dtype=torch.int64, device=dev)
    used = torch.randint(keys // 2, keys + 1, (batch * nk,), generator=g, device=dev).to(torch.int32)
    used[0] = keys
    results = []
    vheads = batch * nk
    merge_blocks = -(-vheads * (nq // nk) // 4) if plan.splits > 1 else 0
    stamps = torch.zeros(vheads * plan.splits * ph.PHASES + merge_blocks * ph.MERGE_PHASES,
                         dtype=torch.int64, device=dev)
    for stamped in (False, True):
        k, v = (c.clone() for c in caches)
        out = torch.full((batch, 1, nq, d), float("nan"), dtype=torch.bfloat16, device=dev)
        args = (qkv.data_ptr(), qkv_splits, qw.data_ptr(), kw.data_ptr(), 1e-6, 1e-6,
                cos.data_ptr(), sin.data_ptr(), position.data_ptr(), k.data_ptr(), v.data_ptr(),
                used.data_ptr(), batch, nq, nk, keys, d ** -0.5, plan.splits, plan.span,
                plan.partials.data_ptr(), plan.stats.data_ptr(), out.data_ptr())
        stream = _lib.stream(torch.device(dev))
        st = (ph._phases_lib()(*args, stamps.data_ptr(), stream) if stamped
              else _lib.lib().qf_decode_attention_qkv(*args, stream))
        assert st == 0, _lib.lib().qf_error_string(st)
        torch.cuda.synchronize()
        results.append((out, k, v))
    for a, b in zip(*results):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    att = stamps[:vheads * plan.splits * ph.PHASES].view(-1, ph.PHASES)[:, :8].cpu()
    assert bool((att > 0).all()) and bool((att[:, 1:] >= att[:, :-1]).all())
    if merge_blocks:
        mer = stamps[vheads * plan.splits * ph.PHASES:].view(-1, ph.MERGE_PHASES)[:, [0, 3, 1, 2]].cpu()
        assert bool((mer > 0).all()) and bool((mer[:, 1:] >= mer[:, :-1]).all())
        assert int(mer[:, 0].min()) >= int(att[:, 0].min())
