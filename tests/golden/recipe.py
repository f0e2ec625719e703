"""Seeded inputs shared by the golden-vector generator and the tests that read its fixtures.

Only outputs are stored in the fixtures; inputs are regenerated from these seeds (CPU torch
generators are deterministic), so the fixtures stay a few tens of KB.
"""

from __future__ import annotations

import zlib

import torch

CONFIG = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=16,
              num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6)
BLOCK_SIZE = 16
PREFILL_PROMPT_LENS = [37, 20, 5]
DECODE_STEPS = 4
CHUNK_PROMPT_LENS = [50, 33]
CHUNK_CUTS = [21, 16]


def _gen(name: str) -> torch.Generator:
    return torch.Generator().manual_seed(zlib.crc32(name.encode()))


def state_dict(shapes: dict[str, tuple[int, ...]]) -> dict[str, torch.Tensor]:
    """bf16 weights by parameter name: norms 1 + N(0, 0.1), lm_head N(0, 1) (untied), the rest N(0, 0.05)."""
    out = {}
    for name, shape in sorted(shapes.items()):
        x = torch.randn(shape, generator=_gen(name))
        if "norm" in name:
            x = 1.0 + 0.1 * x
        elif name != "lm_head.weight":
            x = 0.05 * x
        out[name] = x.to(torch.bfloat16)
    return out


def prompts(lengths, salt: str) -> list[list[int]]:
    g = _gen(salt)
    return [torch.randint(1, CONFIG["vocab_size"], (n,), generator=g).tolist() for n in lengths]


def attend_decode_inputs():
    """q [2,16,1,128], k/v [2,8,40,128] bf16 N(0,1), additive bias for context lengths [40, 23]."""
    g = _gen("attend_decode")
    q = torch.randn(2, 16, 1, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 8, 40, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, 40, 128, generator=g).to(torch.bfloat16)
    allowed = torch.arange(40).view(1, 40) < torch.tensor([[40], [23]])
    bias = torch.zeros(2, 1, 1, 40, dtype=torch.bfloat16)
    bias.masked_fill_(~allowed.view(2, 1, 1, 40), torch.finfo(torch.bfloat16).min)
    return q, k, v, bias


def attend_prefill_inputs():
    """q [1,16,12,128]; k/v [1,8,30,128] = 18 history slots (15 visible) + 12 chunk keys, causal."""
    g = _gen("attend_prefill")
    q = torch.randn(1, 16, 12, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 8, 30, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 8, 30, 128, generator=g).to(torch.bfloat16)
    key = torch.arange(30).view(1, 30)
    query = torch.arange(12).view(12, 1)
    allowed = ((key < 15) | ((key >= 18) & (key - 18 <= query)))
    bias = torch.zeros(1, 1, 12, 30, dtype=torch.bfloat16)
    bias.masked_fill_(~allowed.view(1, 1, 12, 30), torch.finfo(torch.bfloat16).min)
    return q, k, v, bias


__all__ = ["BLOCK_SIZE", "CHUNK_CUTS", "CHUNK_PROMPT_LENS", "CONFIG", "DECODE_STEPS", "PREFILL_PROMPT_LENS",
           "attend_decode_inputs", "attend_prefill_inputs", "prompts", "state_dict"]
