"""Paged-KV runner: chunked prefill with history, prefill store, decode packing and decode step.

Same entry points, arguments and return types as the reference's PagedRunner
(src/mini_infra/worker/paged_runner.py:22-189).  Underneath:

* host metadata is packed with array operations (``worker.metadata``) and uploaded once per call;
* ``run_prefill_chunk_step`` reads the history straight from the pool inside the prefill
  attention kernel -- nothing is gathered -- so ``prefill_cache`` holds the chunk's own K/V
  (``[B, H_kv, padded_chunk_len, D]`` per layer; the reference returns history + chunk, of which
  ``store_prefill`` only ever reads the chunk's tail);
* ``store_prefill`` is one scatter launch for all layers;
* ``run_decode_step`` appends and attends through the pool (see ``model.qwen3``).
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import NamedTuple

import torch

from mini_infra_qwen3_amd.device import StepTimer
from mini_infra_qwen3_amd.model.qwen3 import PagedAttentionMetadata, PagedPrefillMetadata
from mini_infra_qwen3_amd.worker.base_runner import BaseModelRunner, PrefillOutput
from mini_infra_qwen3_amd.worker.kv_cache import KVCache
from mini_infra_qwen3_amd.worker.metadata import pack_decode_rows, pack_prefill_rows, prefill_scatter_indices
from mini_infra_qwen3_amd.worker.paged_kv_cache import PagedKVCachePool
from mini_infra_qwen3_amd.worker.sampler import greedy_sample

_NULL_BLOCK_ID = 0


class PagedDecodeOutput(NamedTuple):
    """Next token per row (input order) and the model time in ms."""

    next_tokens: list[int]
    model_ms: float


class PagedRunner(BaseModelRunner):
    """Stateless runner driving a PagedKVCachePool (reference paged_runner.py:29)."""

    def run_prefill_chunk_step(
        self,
        chunk_token_ids: Sequence[Sequence[int]],
        start_positions: Sequence[int],
        block_tables: Sequence[Sequence[int]],
        pool: PagedKVCachePool,
    ) -> PrefillOutput:
        """Left-padded prefill of prompt chunks whose earlier tokens are already in the pool.

        Row i covers prompt positions ``[start_positions[i], start_positions[i] + len(chunk_token_ids[i]))``;
        its history is the first ``ceil(start / block_size)`` blocks of ``block_tables[i]``, of which the
        first ``start`` slots are visible (reference paged_runner.py:32-102).  next_tokens holds the greedy
        token after each row's last position (meaningful where the chunk completes the prompt).
        """
        packed = torch.from_numpy(pack_prefill_rows(chunk_token_ids, start_positions, block_tables, pool.block_size,
                                                    self.pad_token_id)).to(self.device)
        width = max(len(c) for c in chunk_token_ids)
        input_ids = packed[:, :width]
        position_ids = packed[:, width:2 * width]
        metadata = PagedPrefillMetadata(
            history_block_tables=packed[:, 2 * width + 2:],
            start_lens=packed[:, 2 * width],
            chunk_lens=packed[:, 2 * width + 1],
            kv_pools=tuple(pool.kv_pools),
        )
        with StepTimer(self.device) as timer:
            logits, present = self.model(input_ids, position_ids=position_ids, attn_metadata=metadata,
                                         last_logits_only=True)
            next_token, _ = greedy_sample(logits)
        return PrefillOutput(next_token.squeeze(-1).tolist(), KVCache(present), timer.elapsed_ms)

    def store_prefill(
        self,
        pool: PagedKVCachePool,
        prefill_cache: KVCache,
        block_tables: Sequence[Sequence[int]],
        chunk_lens: Sequence[int],
        start_positions: Sequence[int],
    ) -> None:
        """Writes each row's last ``chunk_lens[i]`` cached tokens to logical positions
        ``start_positions[i]..`` of its block table (reference paged_runner.py:104-136); no sync."""
        index = prefill_scatter_indices(block_tables, chunk_lens, start_positions, prefill_cache.length,
                                        pool.block_size)
        if index.shape[1] == 0:
            return
        index_t = torch.from_numpy(index).to(self.device)
        pool.write_prefill(prefill_cache, token_rows=index_t[0], token_positions=index_t[1], slot_mapping=index_t[2])

    def prepare_decode_inputs(
        self,
        block_tables: Sequence[Sequence[int]],
        last_tokens: Sequence[int],
        positions: Sequence[int],
        block_size: int,
    ) -> tuple[torch.Tensor, torch.Tensor, PagedAttentionMetadata]:
        """Packs one decode step as ``[B, 4 + max_blocks]`` and uploads it once (reference
        paged_runner.py:138-166).  Returns column views: input_ids / position_ids ``[B, 1]`` and the
        metadata's slot_mapping, block_tables and context_lens."""
        packed = torch.from_numpy(pack_decode_rows(block_tables, last_tokens, positions, block_size)).to(self.device)
        metadata = PagedAttentionMetadata(slot_mapping=packed[:, 2], block_tables=packed[:, 4:],
                                          context_lens=packed[:, 3])
        return packed[:, 0:1], packed[:, 1:2], metadata

    def run_decode_step(
        self,
        input_ids: torch.Tensor,
        position_ids: torch.Tensor,
        metadata: PagedAttentionMetadata,
        pool: PagedKVCachePool,
    ) -> PagedDecodeOutput:
        """One decode step: append the new K/V into the pool and attend (reference paged_runner.py:168-189)."""
        with StepTimer(self.device) as timer:
            logits, _ = self.model(input_ids, position_ids=position_ids,
                                   attn_metadata=metadata._replace(kv_pools=tuple(pool.kv_pools)))
            next_token, _ = greedy_sample(logits)
        return PagedDecodeOutput(next_token.squeeze(-1).tolist(), timer.elapsed_ms)


__all__ = ["PagedDecodeOutput", "PagedRunner"]
