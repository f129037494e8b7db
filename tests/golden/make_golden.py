"""Write tests/golden/golden.npz: small input/output vectors of the arithmetic
the reference engine relies on, evaluated with the third-party libraries it
calls (transformers ``Qwen3RMSNorm``, ``apply_rotary_pos_emb``,
``Qwen3RotaryEmbedding``; torch ``F.silu``, ``F.embedding``) on the CPU.

The reference pins transformers==4.51.3 / torch==2.5.1 (requirements.txt:9-11);
this container has transformers 5.15.0 / torch 2.10.0, whose Qwen3 formulas
are textually the same.  Nothing from /root/reference is imported or run.
bf16 arrays are stored as uint16 bit patterns.  Regenerate with
``python tests/golden/make_golden.py``.
"""

from pathlib import Path

import numpy as np
import torch
import transformers
from torch.nn import functional as F
from transformers import Qwen3Config
from transformers.models.qwen3.modeling_qwen3 import (
    Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb)

OUT = Path(__file__).with_name("golden.npz")


def b(t):
    return t.detach().contiguous().view(torch.uint16).numpy()


def normal(shape, mean, std, g):
    return (torch.randn(shape, generator=g) * std + mean).to(torch.bfloat16)


def norm(x, w, eps):
    m = Qwen3RMSNorm(x.shape[-1], eps=eps).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(w)
    return m(x)


def main():
    out = {"meta/transformers": np.array(transformers.__version__),
           "meta/torch": np.array(torch.__version__)}
    with torch.inference_mode():
        # Config 1: x [8,2560] ~ N(0,1), w ~ N(1,0.1), eps 1e-6, seed 0.
        g = torch.Generator().manual_seed(0)
        x = normal((8, 2560), 0.0, 1.0, g)
        w = normal((2560,), 1.0, 0.1, g)
        out.update({"config1_rms_norm/x": b(x), "config1_rms_norm/w": b(w),
                    "config1_rms_norm/eps": np.array(1e-6),
                    "config1_rms_norm/out": b(norm(x, w, 1e-6))})

        cfg = Qwen3Config(head_dim=128, rope_theta=5_000_000, max_position_embeddings=32768,
                          hidden_size=256, num_attention_heads=2, num_key_value_heads=1)
        rot = Qwen3RotaryEmbedding(cfg)
        positions = torch.tensor([0, 1, 2, 511, 2047, 8191, 16383, 32767])
        cos, sin = rot(torch.empty(0, dtype=torch.bfloat16), positions.view(1, -1))
        out.update({"rope_table/inv_freq": rot.inv_freq.numpy(),
                    "rope_table/positions": positions.numpy(),
                    "rope_table/cos": b(cos[0]), "rope_table/sin": b(sin[0])})

        # Module-path Q/K norm + RoPE: 2 sequences at positions 2047 and 32767.
        g = torch.Generator().manual_seed(1)
        q = normal((2, 32, 1, 128), 0.0, 1.0, g)
        k = normal((2, 8, 1, 128), 0.0, 1.0, g)
        qw = normal((128,), 1.0, 0.1, g)
        kw = normal((128,), 1.0, 0.1, g)
        c, s = cos[0, [4, 7]].view(2, 1, 128), sin[0, [4, 7]].view(2, 1, 128)
        oq, ok = apply_rotary_pos_emb(norm(q, qw, 1e-6), norm(k, kw, 3e-6), c, s)
        out.update({"qk_norm_rope/q": b(q)[:, :, 0], "qk_norm_rope/k": b(k)[:, :, 0],
                    "qk_norm_rope/qw": b(qw), "qk_norm_rope/kw": b(kw),
                    "qk_norm_rope/cos": b(c)[:, 0], "qk_norm_rope/sin": b(s)[:, 0],
                    "qk_norm_rope/q_eps": np.array(1e-6), "qk_norm_rope/k_eps": np.array(3e-6),
                    "qk_norm_rope/oq": b(oq)[:, :, 0], "qk_norm_rope/ok": b(ok)[:, :, 0]})

        # SiLU * up with the special values of tests/test_decode_step.py:255.
        g = torch.Generator().manual_seed(2)
        gu = normal((4, 512), 0.0, 4.0, g)
        gu[0, :8] = torch.tensor([-40.0, -12.0, -1.0, 0.0, 1.0, 12.0, 40.0, 88.0])
        gate, up = gu.chunk(2, dim=-1)
        out.update({"silu_mul/gate_up": b(gu), "silu_mul/out": b(F.silu(gate) * up)})

        # Embedding gather.
        g = torch.Generator().manual_seed(3)
        table = normal((64, 64), 0.0, 0.02, g)
        ids = torch.randint(0, 64, (3, 5), generator=g)
        out.update({"embedding/table": b(table), "embedding/ids": ids.numpy(),
                    "embedding/out": b(F.embedding(ids, table))})
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
