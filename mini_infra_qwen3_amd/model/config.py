"""Qwen3 model configuration. Reference src/mini_infra/model/config.py:13-56."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Qwen3Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    torch_dtype: str = "bfloat16"
    tie_word_embeddings: bool = True

    def validate(self) -> None:
        if self.num_attention_heads % self.num_key_value_heads != 0:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")

    @property
    def dtype(self) -> torch.dtype:
        return {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[self.torch_dtype]


def qwen3_0_6b() -> Qwen3Config:
    """Qwen3-0.6B architecture (28 layers, hidden 1024, 16 q / 8 kv heads of 128, vocab 151936)."""
    return Qwen3Config(vocab_size=151936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28,
                       num_attention_heads=16, num_key_value_heads=8, head_dim=128)


__all__ = ["Qwen3Config", "qwen3_0_6b"]
