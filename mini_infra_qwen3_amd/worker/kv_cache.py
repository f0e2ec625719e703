"""Per-layer (key, value) container for prefill caches. Reference src/mini_infra/worker/kv_cache.py:8-52."""

from __future__ import annotations

from collections.abc import Sequence

import torch


class KVCache:
    """Holds one ``(key, value)`` pair per layer, each ``[B, H_kv, L, D]``."""

    def __init__(self, past_key_values: Sequence[tuple[torch.Tensor, torch.Tensor]] | None = None):
        layers = () if past_key_values is None else past_key_values
        self.key_cache: list[torch.Tensor] = [k for k, _ in layers]
        self.value_cache: list[torch.Tensor] = [v for _, v in layers]
        # Not in the reference: the ``[3, N]`` store index (token rows, positions, slots) of the rows
        # the forward already wrote into the pool, or None; a store with the same index has nothing
        # left to do.
        self.written_index = None
        # Not in the reference: for the chunk K/V of a mixed step with ragged rows (one cached row of
        # all the step's chunk tokens), the first token of each chunk row; None otherwise.
        self.ragged_first = None

    @property
    def past_key_values(self) -> list[tuple[torch.Tensor, torch.Tensor]]:
        return list(zip(self.key_cache, self.value_cache))

    @property
    def length(self) -> int:
        """Sequence length L of the cached tensors (0 when empty)."""
        return self.key_cache[0].shape[2] if self.key_cache else 0

    @property
    def total_bytes(self) -> int:
        return sum(k.numel() * k.element_size() + v.numel() * v.element_size()
                   for k, v in zip(self.key_cache, self.value_cache))

    def __len__(self) -> int:
        return len(self.key_cache)

    def __iter__(self):
        return iter(zip(self.key_cache, self.value_cache))

    def __getitem__(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.key_cache[layer_idx], self.value_cache[layer_idx]


__all__ = ["KVCache"]
