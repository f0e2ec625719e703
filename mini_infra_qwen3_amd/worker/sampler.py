"""Greedy sampling of the last position. Reference src/mini_infra/worker/sampler.py:9-23."""

from __future__ import annotations

import torch


def greedy_sample(logits: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """logits ``[B, L, V]`` -> (next_token ``[B, 1]`` int64, last_logits ``[B, V]``)."""
    last_logits = logits[:, -1, :]
    return torch.argmax(last_logits, dim=-1, keepdim=True), last_logits


__all__ = ["greedy_sample"]
