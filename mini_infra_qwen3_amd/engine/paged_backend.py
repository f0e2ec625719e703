"""Step execution of the paged continuous-batching run on the HIP data plane.

Same contract and timing as the reference's PagedScheduleBackend
(src/mini_infra/engine/paged_schedule_backend.py:25-128):

* ``model_ms``: the runner's device-timed forward + greedy sample (StepTimer);
* ``cache_ms``: host-timed, between device syncs: ``store_prefill`` after a prefill step, and
  the decode packing before a decode step; a mixed step (decode rows and prefill chunks in one
  forward, not in the reference) counts both its packing and its store.

The block tables live on the GPU for the whole run (``DeviceBlockTables``, a copy of the
allocator's table matrix kept current by deltas), so a decode step uploads ``[B, 5]`` scalars and
the entries written since the previous step instead of re-packing ``[B, 4 + max_blocks]``
(the reference: src/mini_infra/worker/paged_runner.py:138-166).
"""

from __future__ import annotations

import time
from collections.abc import Sequence
from dataclasses import dataclass

import torch

from mini_infra_qwen3_amd.core import KVCacheManager, PagedCacheConfig, num_blocks_for_tokens, required_pool_blocks
from mini_infra_qwen3_amd.core.scheduler import PrefillChunk, RequestState
from mini_infra_qwen3_amd.core.types import Request
from mini_infra_qwen3_amd.device import synchronize
from mini_infra_qwen3_amd.worker import PagedKVCachePool, PagedRunner
from mini_infra_qwen3_amd.worker.block_tables import DeviceBlockTables


@dataclass(frozen=True)
class ScheduleStepOutput:
    """What one executed step hands back to the loop (reference schedule_backend.py:26-37)."""

    next_tokens: list[int]
    model_ms: float
    cache_ms: float
    physical_batch_size: int
    live_kv_cache_bytes: int
    accessed_kv_cache_tokens: int = 0


class PagedScheduleBackend:
    """Owns the pool and the block allocator; runs prefill chunks and decode steps through PagedRunner."""

    def __init__(self, model: torch.nn.Module, requests: Sequence[Request], max_running_requests: int,
                 paged_cache_config: PagedCacheConfig = PagedCacheConfig(), pad_token_id: int = 0,
                 decode_graphs: bool = False, prefill_graphs: bool = False, prefill_graph_rows: int = 4,
                 mixed_graphs: bool = False, mixed_graph_rows: int = 3, mixed_graph_decode_rows: int = 32,
                 mixed_graph_tokens: int | None = None):
        """``decode_graphs``: capture the decode forward in HIP graphs for every padded (batch, blocks)
        bucket this run can reach, before the run (as serving engines do at start-up).
        ``prefill_graphs``: likewise the chunked-prefill forward of up to ``prefill_graph_rows`` chunks,
        for widths up to the longest prompt and histories up to its blocks.  ``mixed_graphs``: the
        mixed-step forward of up to ``mixed_graph_rows`` chunks (at most ``mixed_graph_tokens`` chunk
        tokens in all: the scheduler's token budget, or no cap) with up to ``mixed_graph_decode_rows``
        decode rows.  A model with reference numerics (``exact``) takes decode graphs per batch size,
        mixed graphs at the padded shapes it runs every mixed step at (``padded_mixed_shape``) and
        no prefill graphs (they pad the chunk width: ValueError)."""
        self.model = model
        self.device = next(model.parameters()).device
        self.block_size = paged_cache_config.block_size
        num_blocks = paged_cache_config.num_blocks or required_pool_blocks(requests, max_running_requests,
                                                                          self.block_size)
        largest = max(num_blocks_for_tokens(r.prompt_len + r.max_new_tokens - 1, self.block_size) for r in requests)
        if largest > num_blocks - 1:
            raise ValueError(f"num_blocks={num_blocks} cannot hold one request of {largest} blocks "
                             "(plus the null block)")
        config = model.config
        self.runner = PagedRunner(model, pad_token_id)
        self.pool = PagedKVCachePool(config.num_hidden_layers, num_blocks, self.block_size,
                                     config.num_key_value_heads, config.head_dim,
                                     next(model.parameters()).dtype, self.device)
        self.kv_cache_manager = KVCacheManager(self.block_size, num_blocks)
        self.tables = DeviceBlockTables(self.kv_cache_manager, min(max_running_requests, len(requests)), largest,
                                        self.device)
        if decode_graphs:
            self.runner.enable_decode_graphs(self.pool, max_batch=min(max_running_requests, len(requests)),
                                             max_blocks=largest, tables=self.tables)
        longest = max(r.prompt_len for r in requests)
        if mixed_graphs:
            self.runner.enable_mixed_graphs(
                self.pool, max_rows=min(mixed_graph_rows, max_running_requests), max_width=longest,
                max_chunk_tokens=mixed_graph_tokens,
                max_decode_rows=min(mixed_graph_decode_rows, max_running_requests, len(requests)),
                max_history_blocks=num_blocks_for_tokens(longest, self.block_size), max_decode_blocks=largest)
        if prefill_graphs:
            self.runner.enable_prefill_graphs(self.pool, max_rows=min(prefill_graph_rows, max_running_requests),
                                              max_width=longest,
                                              max_history_blocks=num_blocks_for_tokens(longest, self.block_size))

    def _live_bytes(self) -> int:
        return self.kv_cache_manager.num_used_blocks * self.pool.bytes_per_block

    def execute_prefill(self, chunks: Sequence[PrefillChunk]) -> ScheduleStepOutput:
        tables = [self.kv_cache_manager.block_table(c.state.request.request_idx) for c in chunks]
        starts = [c.start for c in chunks]
        out = self.runner.run_prefill_chunk_step([c.state.request.token_ids[c.start:c.end] for c in chunks], starts,
                                                 tables, self.pool)
        synchronize(self.device)
        t0 = time.perf_counter()
        self.runner.store_prefill(self.pool, out.prefill_cache, tables, [c.num_tokens for c in chunks], starts)
        synchronize(self.device)
        cache_ms = (time.perf_counter() - t0) * 1000.0
        return ScheduleStepOutput([t for t, c in zip(out.next_tokens, chunks) if c.is_last], out.model_ms, cache_ms,
                                  len(chunks), self._live_bytes(), sum(c.start for c in chunks))

    def execute_decode(self, states: Sequence[RequestState]) -> ScheduleStepOutput:
        synchronize(self.device)
        t0 = time.perf_counter()
        ids, pos, meta = self.runner.prepare_decode_from_tables(
            self.tables, [s.request.request_idx for s in states], last_tokens=[s.generated[-1] for s in states],
            positions=[s.cache_length for s in states])
        synchronize(self.device)
        cache_ms = (time.perf_counter() - t0) * 1000.0
        out = self.runner.run_decode_step(ids, pos, meta, self.pool)
        return ScheduleStepOutput(out.next_tokens, out.model_ms, cache_ms, len(states), self._live_bytes(),
                                  sum(s.cache_length + 1 for s in states))

    def execute_mixed(self, states: Sequence[RequestState], chunks: Sequence[PrefillChunk]) -> ScheduleStepOutput:
        """Decode rows ``states`` and prefill ``chunks`` in one forward; tokens: the decode rows', then
        those of the chunks that complete their prompt."""
        manager = self.kv_cache_manager
        tables = [manager.block_table(c.state.request.request_idx) for c in chunks]
        starts = [c.start for c in chunks]
        synchronize(self.device)
        t0 = time.perf_counter()
        ids, pos, meta = self.runner.prepare_mixed_inputs(
            [c.state.request.token_ids[c.start:c.end] for c in chunks], starts, tables,
            [s.generated[-1] for s in states], [s.cache_length for s in states],
            [manager.block_table(s.request.request_idx) for s in states], self.pool)
        synchronize(self.device)
        cache_ms = (time.perf_counter() - t0) * 1000.0
        out = self.runner.run_mixed_step(ids, pos, meta)
        synchronize(self.device)
        t0 = time.perf_counter()
        self.runner.store_prefill(self.pool, out.prefill_cache, tables, [c.num_tokens for c in chunks], starts)
        synchronize(self.device)
        cache_ms += (time.perf_counter() - t0) * 1000.0
        tokens = out.decode_next_tokens + [t for t, c in zip(out.prefill_next_tokens, chunks) if c.is_last]
        return ScheduleStepOutput(tokens, out.model_ms, cache_ms, len(states) + len(chunks), self._live_bytes(),
                                  sum(s.cache_length + 1 for s in states) + sum(c.start for c in chunks))


__all__ = ["PagedScheduleBackend", "ScheduleStepOutput"]
