"""Greedy sampling of the last position. Reference src/mini_infra/worker/sampler.py:9-23."""

from __future__ import annotations

import torch

from mini_infra_qwen3_amd.data_plane import argmax_rows


def greedy_sample(logits: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 logits ``[B, L, V]`` on the GPU -> (next_token ``[B, 1]`` int64, last_logits ``[B, V]``).

    The argmax is the HIP kernel behind ``argmax_rows`` (torch.argmax's answer: first index on ties).
    """
    last_logits = logits[:, -1, :]
    return argmax_rows(last_logits).unsqueeze(-1), last_logits


__all__ = ["greedy_sample"]
