"""Whole-prompt prefill runner. Reference src/mini_infra/worker/base_runner.py:18-86."""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any, NamedTuple

import torch

from mini_infra_qwen3_amd.device import StepTimer
from mini_infra_qwen3_amd.worker.kv_cache import KVCache
from mini_infra_qwen3_amd.worker.sampler import greedy_sample


class PrefillOutput(NamedTuple):
    """First token per row, the prefill K/V (per layer ``[B, H_kv, L, D]``) and the model time in ms."""

    next_tokens: list[int]
    prefill_cache: KVCache
    model_ms: float


def _left_pad_sequences(token_sequences: Sequence[Any], pad_token_id: int, device: torch.device):
    """Left-pads 1-d token sequences into ``(input_ids, attention_mask, position_ids, lengths)``.

    Same contract as the reference helper (base_runner.py:26-60): real tokens at the end of each
    row, mask True on them, positions 0.. on real tokens and 0 on padding.  Built on the host and
    uploaded once.
    """
    if not token_sequences:
        raise ValueError("token_sequences must not be empty")
    rows = [list(map(int, s)) for s in token_sequences]
    if any(len(r) < 1 for r in rows):
        raise ValueError("every prompt must be a non-empty 1-d token sequence")
    width = max(len(r) for r in rows)
    ids = torch.full((len(rows), width), pad_token_id, dtype=torch.long)
    mask = torch.zeros((len(rows), width), dtype=torch.bool)
    pos = torch.zeros((len(rows), width), dtype=torch.long)
    for i, r in enumerate(rows):
        n = len(r)
        ids[i, width - n:] = torch.tensor(r, dtype=torch.long)
        mask[i, width - n:] = True
        pos[i, width - n:] = torch.arange(n)
    lengths = torch.tensor([len(r) for r in rows], dtype=torch.long)
    return ids.to(device), mask.to(device), pos.to(device), lengths.to(device)


class BaseModelRunner:
    """Holds the model and device; runs whole-prompt prefill (no history)."""

    def __init__(self, model: torch.nn.Module, pad_token_id: int = 0):
        self.model = model
        self.device = next(model.parameters()).device
        self.pad_token_id = pad_token_id

    def run_prefill_step(self, prompt_sequences: Sequence[Sequence[int]]) -> PrefillOutput:
        """Left-padded prefill of new prompts: first token, prefill K/V and model time."""
        input_ids, attention_mask, position_ids, _ = _left_pad_sequences(prompt_sequences, self.pad_token_id,
                                                                         self.device)
        with StepTimer(self.device) as timer:
            logits, present = self.model(input_ids, attention_mask=attention_mask, position_ids=position_ids,
                                         last_logits_only=True)
            next_token, _ = greedy_sample(logits)
        return PrefillOutput(next_token.squeeze(-1).tolist(), KVCache(present), timer.elapsed_ms)


__all__ = ["BaseModelRunner", "PrefillOutput"]
