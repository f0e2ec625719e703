"""Paged-KV runner: chunked prefill with history, prefill store, decode packing and decode step.

Same entry points, arguments and return types as the reference's PagedRunner
(src/mini_infra/worker/paged_runner.py:22-189).  Underneath:

* host metadata is packed with array operations (``worker.metadata``) and uploaded once per call;
* ``run_prefill_chunk_step`` reads the history straight from the pool inside the prefill
  attention kernel -- nothing is gathered -- so ``prefill_cache`` holds the chunk's own K/V
  (``[B, H_kv, padded_chunk_len, D]`` per layer; the reference returns history + chunk, of which
  ``store_prefill`` only ever reads the chunk's tail);
* ``store_prefill`` is one scatter launch for all layers;
* ``run_decode_step`` appends and attends through the pool (see ``model.qwen3``).  With
  ``enable_decode_graphs`` the whole decode forward is captured once per padded (batch, blocks)
  bucket in a HIP graph: ``prepare_decode_inputs`` then packs the step (pad rows: slot -1 = no
  append, context 0 = zero output) straight into the bucket's static metadata buffer with one
  upload, and ``run_decode_step`` replays the graph -- one launch instead of ~300.  A model with
  reference numerics (``exact``) gets one graph per batch size instead (a GEMM's rows can change
  with its M, so padding the batch would change them) and one table width (the decode kernel
  reads only the blocks a row's context covers); prefill graphs, which pad the chunk width, are
  for models without reference numerics.  Such a model runs every mixed step at a padded shape
  (``padded_mixed_shape``), so mixed graphs serve it as well;
* ``prepare_mixed_inputs`` / ``run_mixed_step`` run prefill chunks and decode tokens in one forward
  (the mixed batching the reference plans next: src/mini_infra/core/scheduler.py:310-311).

A graph bucket's static buffers hold one prepared step, so with graphs each ``prepare_*`` call is
followed by its ``run_*`` call before the next ``prepare_*`` of the same kind (as the reference's
loop calls them); eager steps carry everything in the tensors and metadata they return.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import NamedTuple

import numpy as np
import torch

from mini_infra_qwen3_amd.data_plane import argmax_rows
from mini_infra_qwen3_amd.device import StepTimer
from mini_infra_qwen3_amd.model.qwen3 import PagedAttentionMetadata, PagedMixedMetadata, PagedPrefillMetadata
from mini_infra_qwen3_amd.worker.base_runner import BaseModelRunner, PrefillOutput
from mini_infra_qwen3_amd.worker.block_tables import DeviceBlockTables
from mini_infra_qwen3_amd.worker.kv_cache import KVCache
from mini_infra_qwen3_amd.worker.metadata import (MIXED_WIDTH_QUANTUM, pack_decode_rows, pack_mixed_rows,
                                                  pack_prefill_rows, padded_mixed_shape, prefill_scatter_indices)
from mini_infra_qwen3_amd.worker.paged_kv_cache import PagedKVCachePool
from mini_infra_qwen3_amd.worker.sampler import greedy_sample

_NULL_BLOCK_ID = 0


class _DecodeGraph:
    """The decode forward of one padded bucket, captured over a static packed-metadata buffer
    ``[batch, 4 + blocks]`` (token, position, slot, context length, block table) -- or, over a
    persistent ``DeviceBlockTables``, ``[batch, 5]`` (token, position, slot, context length, table
    row), the block tables being gathered from the device copy inside the graph."""

    def __init__(self, model: torch.nn.Module, pool: PagedKVCachePool, batch: int, blocks: int,
                 device: torch.device, tables: DeviceBlockTables | None = None):
        self.batch, self.blocks = batch, blocks
        self.tables = tables
        self.static = torch.zeros((batch, 5 if tables is not None else 4 + blocks), dtype=torch.long, device=device)
        self.static[:, 2] = -1  # every row is padding until a step is loaded
        self._staging = torch.empty(tuple(self.static.shape), dtype=torch.long, pin_memory=True)
        self._copied = torch.cuda.Event()  # the last copy out of the staging buffer
        self._views: dict[int, tuple] = {}
        ids, pos, meta = self.views(batch)
        meta = meta._replace(kv_pools=tuple(pool.kv_pools))
        side = torch.cuda.Stream(device)  # default priority
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(2):  # warm-up outside the capture: GEMM choices, library state
                model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.inference_mode():
            logits, _ = model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
        self.logits = logits[:, -1]

    def views(self, rows: int):
        """(input_ids, position_ids, metadata) of the first ``rows`` rows (built once per row count)."""
        cached = self._views.get(rows)
        if cached is None:
            cached = self._views[rows] = self._make_views(rows)
        return cached

    def _make_views(self, rows: int):
        s = self.static[:rows]
        if self.tables is not None:
            return s[:, 0:1], s[:, 1:2], PagedAttentionMetadata(slot_mapping=s[:, 2], block_tables=self.tables.tensor,
                                                                context_lens=s[:, 3], table_rows=s[:, 4])
        return s[:, 0:1], s[:, 1:2], PagedAttentionMetadata(slot_mapping=s[:, 2], block_tables=s[:, 4:],
                                                            context_lens=s[:, 3])

    def load(self, packed: np.ndarray) -> None:
        """Copies a step packed at the bucket's shape (``pack_decode_rows(..., rows, blocks)``, or the
        ``[batch, 5]`` rows of a table-backed graph) through pinned memory (the copy is ordered before
        the replay on the same stream; the host waits for the previous copy before reusing the buffer)."""
        self._copied.synchronize()
        self._staging.numpy()[...] = packed
        self.static.copy_(self._staging, non_blocking=True)
        self._copied.record()


class _PrefillGraph:
    """The chunked-prefill forward of one (rows, padded width W) bucket with history tables NB blocks
    wide, captured over a static packed buffer ``[rows, 2 W + 2 + NB + W]`` in the
    ``pack_prefill_rows(..., slots=True)`` layout.  The chunk K/V (the present) go to the runner's
    staging buffers, which every prefill graph shares, so captured graphs hold no per-graph outputs
    beyond their logits; tokens with a slot (>= 0) also go straight into the pool."""

    def __init__(self, model: torch.nn.Module, pool: PagedKVCachePool, rows: int, width: int, hist_blocks: int,
                 staging: torch.Tensor, mempool, pad_token_id: int, device: torch.device):
        self.rows, self.width, self.hist_blocks = rows, width, hist_blocks
        self.pad_token_id = pad_token_id
        self.static = torch.zeros((rows, 3 * width + 2 + hist_blocks), dtype=torch.long, device=device)
        self.static[:, :width] = pad_token_id  # every row is an empty chunk until a step is loaded
        self.static[:, 2 * width + 2 + hist_blocks:] = -1
        ids, pos, meta = self.views()
        tokens = rows * width
        meta = meta._replace(kv_pools=tuple(pool.kv_pools),
                             kv_out=tuple((staging[l, 0, :tokens], staging[l, 1, :tokens])
                                          for l in range(staging.shape[0])))
        side = torch.cuda.Stream(device)  # default priority
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(2):  # warm-up outside the capture: GEMM choices, library state
                model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=mempool), torch.inference_mode():
            logits, presents = model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
        self.logits = logits[:, -1]
        self.presents = presents

    def views(self):
        s, w, nb = self.static, self.width, self.hist_blocks
        return s[:, :w], s[:, w:2 * w], PagedPrefillMetadata(history_block_tables=s[:, 2 * w + 2:2 * w + 2 + nb],
                                                             start_lens=s[:, 2 * w], chunk_lens=s[:, 2 * w + 1],
                                                             slot_mapping=s[:, 2 * w + 2 + nb:])

    def load(self, packed: np.ndarray) -> None:
        """Copies a step packed at the bucket's shape (``pack_prefill_rows(..., width, history_blocks,
        slots=True)``)."""
        self.static.copy_(torch.from_numpy(packed))


class _MixedGraph:
    """A mixed step's forward for one (chunk rows P, chunk tokens C, decode rows D) bucket, with
    history tables NB and decode tables MB blocks wide, captured over a static buffer in the
    ``pack_mixed_rows`` layout (ragged chunk rows); the attention sees each chunk row left-padded
    to ``width``, the longest chunk the graph serves (query tiles wholly in a row's padding exit at
    once).  The step's K/V (chunk and decode tokens) go to the shared staging buffers.  Pad decode
    rows carry slot -1 (no append) and context 0 (zero output); pad chunk tokens belong to no row."""

    def __init__(self, model: torch.nn.Module, pool: PagedKVCachePool, rows: int, chunk_tokens: int, width: int,
                 decode_rows: int, hist_blocks: int, decode_blocks: int, staging: torch.Tensor, mempool,
                 pad_token_id: int, device: torch.device):
        self.rows, self.chunk_tokens, self.width, self.decode_rows = rows, chunk_tokens, width, decode_rows
        self.hist_blocks, self.decode_blocks = hist_blocks, decode_blocks
        self.pad_token_id = pad_token_id
        self.tokens = chunk_tokens + decode_rows
        self.static = torch.from_numpy(self._empty()).to(device)
        ids, pos, meta = self.views()
        t = self.tokens
        meta = meta._replace(kv_pools=tuple(pool.kv_pools),
                             prefill=meta.prefill._replace(kv_out=tuple((staging[l, 0, :t], staging[l, 1, :t])
                                                                        for l in range(staging.shape[0]))))
        side = torch.cuda.Stream(device)  # default priority
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(2):  # warm-up outside the capture: GEMM choices, library state
                model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=mempool), torch.inference_mode():
            logits, presents = model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
        self.logits = logits[:, -1]
        self.presents = presents
        self.static_slots_ptr = self.views()[2].decode.slot_mapping.data_ptr()

    def _empty(self) -> np.ndarray:
        t = self.tokens
        full = np.zeros(2 * t + self.rows * (3 + self.hist_blocks) + self.decode_rows * (2 + self.decode_blocks),
                        dtype=np.int64)
        full[:t] = self.pad_token_id  # chunk rows of length 0: nothing to attend or store
        dec = full[2 * t + self.rows * (3 + self.hist_blocks):].reshape(self.decode_rows, 2 + self.decode_blocks)
        dec[:, 0] = -1
        return full

    def views(self):
        s, t = self.static, self.tokens
        at = 2 * t + self.rows * (3 + self.hist_blocks)
        chunk = s[2 * t:at].view(self.rows, 3 + self.hist_blocks)
        dec = s[at:].view(self.decode_rows, 2 + self.decode_blocks)
        meta = PagedMixedMetadata(
            prefill=PagedPrefillMetadata(history_block_tables=chunk[:, 3:], start_lens=chunk[:, 0],
                                         chunk_lens=chunk[:, 1]),
            decode=PagedAttentionMetadata(slot_mapping=dec[:, 0], block_tables=dec[:, 2:], context_lens=dec[:, 1]),
            prefill_rows=self.rows, prefill_width=self.width, chunk_first=chunk[:, 2],
            chunk_tokens=self.chunk_tokens)
        return s[:t].view(1, t), s[t:2 * t].view(1, t), meta

    def load(self, flat: np.ndarray) -> None:
        """Copies a step packed at the bucket's shape (``pack_mixed_rows`` with its four sizes)."""
        self.static.copy_(torch.from_numpy(flat))


class PagedDecodeOutput(NamedTuple):
    """Next token per row (input order) and the model time in ms."""

    next_tokens: list[int]
    model_ms: float


class MixedStepOutput(NamedTuple):
    """A mixed step: the greedy token after each chunk row (meaningful where the chunk completes its
    prompt) and after each decode row, the chunks' K/V (for ``store_prefill``) and the model time."""

    prefill_next_tokens: list[int]
    decode_next_tokens: list[int]
    prefill_cache: KVCache
    model_ms: float


class PagedRunner(BaseModelRunner):
    """Runner driving a PagedKVCachePool (reference paged_runner.py:29); stateless unless decode
    graphs are enabled."""

    def __init__(self, model: torch.nn.Module, pad_token_id: int = 0):
        super().__init__(model, pad_token_id)
        self._graphs: dict[tuple[int, int], _DecodeGraph] = {}
        self._graph_pool: PagedKVCachePool | None = None
        self._graph_tables: DeviceBlockTables | None = None
        self._batch_buckets: list[int] = []
        self._block_buckets: list[int] = []
        self._loaded: tuple[_DecodeGraph, int] | None = None
        self._prefill_graphs: dict[tuple[int, int], _PrefillGraph] = {}
        self._prefill_pool: PagedKVCachePool | None = None
        self._width_quantum, self._hist_blocks = 1, 0
        self._mixed_graphs: dict[tuple[int, int, int], _MixedGraph] = {}
        self._mixed_pool: PagedKVCachePool | None = None
        self._mixed_loaded: tuple[_MixedGraph, int] | None = None
        self._mixed_width = 0
        self._decode_row_buckets: list[int] = []
        self._staging: torch.Tensor | None = None
        self._mempool = None

    def _shared_staging(self, tokens: int, pool: PagedKVCachePool) -> torch.Tensor:
        """Chunk K/V staging ``[layers, 2, tokens, H_kv, D]`` shared by the prefill and mixed graphs
        (a larger request allocates a new one; graphs captured earlier keep theirs alive)."""
        if self._staging is None or self._staging.shape[2] < tokens:
            cfg = self.model.config
            self._staging = torch.empty((cfg.num_hidden_layers, 2, tokens, cfg.num_key_value_heads, cfg.head_dim),
                                        dtype=pool.storage.dtype, device=self.device)
        if self._mempool is None:
            self._mempool = torch.cuda.graph_pool_handle()
        return self._staging

    def enable_decode_graphs(self, pool: PagedKVCachePool, max_batch: int, max_blocks: int,
                             batch_buckets: Sequence[int] | None = None, block_quantum: int = 16,
                             tables: DeviceBlockTables | None = None) -> None:
        """Captures the decode forward for every (batch bucket, block bucket) up to ``max_batch``
        rows and ``max_blocks`` blocks per row, over ``pool``.  Steps outside the buckets, or on
        another pool, run without a graph.  With ``tables``, the graphs read the block tables from
        that persistent device copy (one table width) and serve ``prepare_decode_from_tables``."""
        if self.device.type != "cuda":
            raise RuntimeError("decode graphs need the GPU")
        exact = getattr(self.model, "exact", False)
        if tables is not None:
            max_blocks = tables.tensor.shape[1]
        if exact or tables is not None:  # one table width
            block_quantum = max(int(max_blocks), 1)
        if exact:  # every batch size its own graph (no padded rows in the GEMMs)
            batch_buckets = range(1, max_batch + 1)
        elif batch_buckets is None:
            batch_buckets = [b for b in (1, 2, 4, 8, 12, 16, 24, 32, 48, 64, 80, 96, 112, 128, 160, 192, 224, 256)
                             if b < max_batch] + [max_batch]
        self._batch_buckets = sorted(set(int(b) for b in batch_buckets if 0 < b <= max_batch))
        top = -(-max_blocks // block_quantum) * block_quantum
        self._block_buckets = list(range(block_quantum, top + 1, block_quantum))
        self._graph_pool = pool
        self._graph_tables = tables
        self._graphs = {}
        for b in self._batch_buckets:
            for nb in self._block_buckets:
                self._graphs[(b, nb)] = _DecodeGraph(self.model, pool, b, nb, self.device, tables)
        torch.cuda.synchronize(self.device)

    def enable_prefill_graphs(self, pool: PagedKVCachePool, max_rows: int, max_width: int, max_history_blocks: int,
                              width_quantum: int = 128) -> None:
        """Captures the chunked-prefill forward for 1..``max_rows`` rows and padded chunk widths in
        multiples of ``width_quantum`` up to ``max_width``, over ``pool``.  Every graph takes history
        tables ``max_history_blocks`` wide (null-padded; the kernel reads only the entries a row's
        start covers, so the width costs nothing).  Steps outside the buckets, or on another pool,
        run without a graph.  With graphs, a step's ``prefill_cache`` lives in buffers the next
        graphed prefill step overwrites: store it first (as ``store_prefill`` right after the step
        does)."""
        if self.device.type != "cuda":
            raise RuntimeError("prefill graphs need the GPU")
        self._refuse_padded_graphs("prefill")
        top_w = -(-max_width // width_quantum) * width_quantum
        staging = self._shared_staging(max_rows * top_w, pool)
        self._prefill_pool = pool
        self._width_quantum, self._hist_blocks = width_quantum, max(int(max_history_blocks), 0)
        self._prefill_graphs = {}
        for rows in range(1, max_rows + 1):
            for width in range(width_quantum, top_w + 1, width_quantum):
                self._prefill_graphs[(rows, width)] = _PrefillGraph(
                    self.model, pool, rows, width, self._hist_blocks, staging, self._mempool, self.pad_token_id,
                    self.device)
        torch.cuda.synchronize(self.device)

    def enable_mixed_graphs(self, pool: PagedKVCachePool, max_rows: int, max_width: int, max_decode_rows: int,
                            max_history_blocks: int, max_decode_blocks: int, width_quantum: int = MIXED_WIDTH_QUANTUM,
                            decode_row_buckets: Sequence[int] | None = None,
                            max_chunk_tokens: int | None = None) -> None:
        """Captures the mixed-step forward for 1..``max_rows`` chunk rows of at most ``max_width``
        tokens each, chunk tokens (ragged rows, back to back) in multiples of ``width_quantum`` up to
        the rows times ``max_width`` (capped at ``max_chunk_tokens``) rounded up, and decode-row
        buckets up to ``max_decode_rows`` (pad rows append nothing), with history / decode tables
        ``max_history_blocks`` / ``max_decode_blocks`` wide, over ``pool``.  Other steps run without a
        graph; as with prefill graphs, store a step's ``prefill_cache`` before the next graphed step.
        A model with reference numerics runs every mixed step at ``padded_mixed_shape`` (graphed or
        not), so its buckets are exactly those shapes: chunk-token quantum ``MIXED_WIDTH_QUANTUM`` and
        power-of-two decode rows."""
        if self.device.type != "cuda":
            raise RuntimeError("mixed graphs need the GPU")
        exact = getattr(self.model, "exact", False)
        if decode_row_buckets is None:
            decode_row_buckets = [b for b in (1, 2, 4, 8, 16, 32, 64, 128, 256) if b < max_decode_rows]
            if not exact:
                decode_row_buckets.append(max_decode_rows)
            elif max_decode_rows & (max_decode_rows - 1) == 0:
                decode_row_buckets.append(max_decode_rows)
        if exact and (width_quantum != MIXED_WIDTH_QUANTUM or
                      any(int(b) & (int(b) - 1) for b in decode_row_buckets if int(b) > 0)):
            raise ValueError(f"a model with reference numerics runs mixed steps at chunk-token multiples of "
                             f"{MIXED_WIDTH_QUANTUM} and power-of-two decode rows; its graphs must use those buckets")
        self._decode_row_buckets = sorted(set(int(b) for b in decode_row_buckets if 0 < b <= max_decode_rows))
        def top(rows: int) -> int:
            tokens = rows * max_width if max_chunk_tokens is None else min(rows * max_width, max_chunk_tokens)
            return -(-tokens // width_quantum) * width_quantum

        top_c = top(max_rows)
        staging = self._shared_staging(top_c + max(self._decode_row_buckets, default=0), pool)
        self._mixed_pool = pool
        self._mixed_quantum = width_quantum
        self._mixed_width = int(max_width)
        self._mixed_tables = (max(int(max_history_blocks), 0), max(int(max_decode_blocks), 1))
        self._mixed_graphs = {}
        for rows in range(1, max_rows + 1):
            for c in range(width_quantum, top(rows) + 1, width_quantum):
                for d in self._decode_row_buckets:
                    self._mixed_graphs[(rows, c, d)] = _MixedGraph(
                        self.model, pool, rows, c, self._mixed_width, d, *self._mixed_tables, staging,
                        self._mempool, self.pad_token_id, self.device)
        torch.cuda.synchronize(self.device)

    def _refuse_padded_graphs(self, kind: str) -> None:
        if getattr(self.model, "exact", False):
            raise ValueError(f"{kind} graphs pad the chunk width, which changes the GEMMs' M and with it the bits of "
                             "their rows: a model with reference numerics (exact) runs these steps without graphs")

    def _mixed_bucket(self, rows: int, width: int, chunk_tokens: int, hist_blocks: int, decode_rows: int,
                      decode_blocks: int) -> _MixedGraph | None:
        if not self._mixed_graphs or hist_blocks > self._mixed_tables[0] or decode_blocks > self._mixed_tables[1] \
                or width > self._mixed_width:
            return None
        d = next((b for b in self._decode_row_buckets if b >= decode_rows), None)
        c = -(-chunk_tokens // self._mixed_quantum) * self._mixed_quantum
        return None if d is None else self._mixed_graphs.get((rows, c, d))

    def _prefill_bucket(self, rows: int, width: int, blocks: int) -> _PrefillGraph | None:
        if blocks > self._hist_blocks:
            return None
        return self._prefill_graphs.get((rows, -(-width // self._width_quantum) * self._width_quantum))

    def _bucket(self, rows: int, blocks: int) -> _DecodeGraph | None:
        b = next((x for x in self._batch_buckets if x >= rows), None)
        nb = next((x for x in self._block_buckets if x >= blocks), None)
        return None if b is None or nb is None else self._graphs[(b, nb)]

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
        width = max(len(c) for c in chunk_token_ids)
        graph = None
        if self._prefill_graphs and pool is self._prefill_pool:
            hist = max(-(-st // pool.block_size) for st in start_positions)
            graph = self._prefill_bucket(len(chunk_token_ids), width, hist)
        # When every table already covers its chunk (the reference's contract allows it:
        # paged_runner.py:49), q/k norm + RoPE also writes the chunk's K/V rows into their slots and
        # the store that follows has nothing left to do.
        lens = [len(c) for c in chunk_token_ids]
        direct = all(len(t) * pool.block_size >= s + n for t, s, n in zip(block_tables, start_positions, lens))
        if graph is not None:
            packed = pack_prefill_rows(chunk_token_ids, start_positions, block_tables, pool.block_size,
                                       self.pad_token_id, width=graph.width, history_blocks=graph.hist_blocks,
                                       slots=True)
            if not direct:
                packed[:, 2 * graph.width + 2 + graph.hist_blocks:] = -1
            graph.load(packed)
            with StepTimer(self.device) as timer:
                graph.graph.replay()
                next_token = argmax_rows(graph.logits)
            cache = KVCache(graph.presents)
            if direct:
                cache.written_index = prefill_scatter_indices(block_tables, lens, start_positions, graph.width,
                                                              pool.block_size)
            return PrefillOutput(next_token.tolist(), cache, timer.elapsed_ms)
        packed_np = pack_prefill_rows(chunk_token_ids, start_positions, block_tables, pool.block_size,
                                      self.pad_token_id, slots=direct)
        nb = packed_np.shape[1] - 2 * width - 2 - (width if direct else 0)
        packed = torch.from_numpy(packed_np).to(self.device)
        input_ids = packed[:, :width]
        position_ids = packed[:, width:2 * width]
        metadata = PagedPrefillMetadata(
            history_block_tables=packed[:, 2 * width + 2:2 * width + 2 + nb],
            start_lens=packed[:, 2 * width],
            chunk_lens=packed[:, 2 * width + 1],
            kv_pools=tuple(pool.kv_pools),
            slot_mapping=packed[:, 2 * width + 2 + nb:] if direct else None,
        )
        with StepTimer(self.device) as timer:
            logits, present = self.model(input_ids, position_ids=position_ids, attn_metadata=metadata,
                                         last_logits_only=True)
            next_token, _ = greedy_sample(logits)
        cache = KVCache(present)
        if direct:
            cache.written_index = prefill_scatter_indices(block_tables, lens, start_positions, width, pool.block_size)
        return PrefillOutput(next_token.squeeze(-1).tolist(), cache, timer.elapsed_ms)

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
                                        pool.block_size, row_first=getattr(prefill_cache, "ragged_first", None))
        if index.shape[1] == 0:
            return
        written = getattr(prefill_cache, "written_index", None)
        if written is not None and written.shape == index.shape and np.array_equal(written, index):
            return  # the forward already wrote these rows into these slots
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
        graph = None
        if self._graphs and self._graph_tables is None and block_size == self._graph_pool.block_size:
            graph = self._bucket(len(block_tables), max((len(t) for t in block_tables), default=0))
        self._loaded = None
        if graph is not None:
            graph.load(pack_decode_rows(block_tables, last_tokens, positions, block_size, rows=graph.batch,
                                        blocks=graph.blocks))
            self._loaded = (graph, len(block_tables))
            return graph.views(len(block_tables))
        rows = pack_decode_rows(block_tables, last_tokens, positions, block_size)
        packed = torch.from_numpy(rows).to(self.device)
        metadata = PagedAttentionMetadata(slot_mapping=packed[:, 2], block_tables=packed[:, 4:],
                                          context_lens=packed[:, 3])
        return packed[:, 0:1], packed[:, 1:2], metadata

    def prepare_decode_from_tables(
        self,
        tables: DeviceBlockTables,
        request_ids: Sequence[int],
        last_tokens: Sequence[int],
        positions: Sequence[int],
    ) -> tuple[torch.Tensor, torch.Tensor, PagedAttentionMetadata]:
        """``prepare_decode_inputs`` for requests whose block tables live in ``tables`` (and its
        manager): brings the device copy up to date with the manager's new entries, then uploads
        ``[B, 5]`` (token, position, slot, context length, table row) -- no table is re-packed.
        Slots come from the manager's matrix on the host: ``table[pos // bs] * bs + pos % bs``."""
        manager = tables.manager
        bs = manager.block_size
        batch = len(request_ids)
        rows = np.fromiter((manager.row_of(r) for r in request_ids), dtype=np.int64, count=batch)
        pos = np.asarray(positions, dtype=np.int64)
        slots = manager.table_matrix[rows, pos // bs] * bs + pos % bs
        packed = np.stack((np.asarray(last_tokens, dtype=np.int64), pos, slots, pos + 1, rows), axis=1)
        tables.sync()
        self._loaded = None
        graph = None
        if self._graphs and tables is self._graph_tables:
            graph = self._bucket(batch, tables.tensor.shape[1])
        if graph is not None:
            full = np.zeros((graph.batch, 5), dtype=np.int64)
            full[:, 2] = -1  # pad rows: no append, context 0 (zero output)
            full[:batch] = packed
            graph.load(full)
            self._loaded = (graph, batch)
            return graph.views(batch)
        dev = torch.from_numpy(packed).to(self.device)
        metadata = PagedAttentionMetadata(slot_mapping=dev[:, 2], block_tables=tables.tensor, context_lens=dev[:, 3],
                                          table_rows=dev[:, 4])
        return dev[:, 0:1], dev[:, 1:2], metadata

    def run_decode_step(
        self,
        input_ids: torch.Tensor,
        position_ids: torch.Tensor,
        metadata: PagedAttentionMetadata,
        pool: PagedKVCachePool,
    ) -> PagedDecodeOutput:
        """One decode step: append the new K/V into the pool and attend (reference paged_runner.py:168-189)."""
        loaded = self._loaded
        if (loaded is not None and pool is self._graph_pool and input_ids.shape[0] == loaded[1]
                and metadata.slot_mapping.data_ptr() == loaded[0].static[:, 2].data_ptr()):
            graph, rows = loaded
            with StepTimer(self.device) as timer:
                graph.graph.replay()
                next_token = argmax_rows(graph.logits[:rows])
            return PagedDecodeOutput(next_token.tolist(), timer.elapsed_ms)
        with StepTimer(self.device) as timer:
            logits, _ = self.model(input_ids, position_ids=position_ids,
                                   attn_metadata=metadata._replace(kv_pools=tuple(pool.kv_pools)))
            next_token, _ = greedy_sample(logits)
        return PagedDecodeOutput(next_token.squeeze(-1).tolist(), timer.elapsed_ms)

    def prepare_mixed_inputs(
        self,
        chunk_token_ids: Sequence[Sequence[int]],
        start_positions: Sequence[int],
        prefill_block_tables: Sequence[Sequence[int]],
        last_tokens: Sequence[int],
        positions: Sequence[int],
        decode_block_tables: Sequence[Sequence[int]],
        pool: PagedKVCachePool,
    ) -> tuple[torch.Tensor, torch.Tensor, PagedMixedMetadata]:
        """Packs a mixed step -- chunk rows as ``run_prefill_chunk_step`` takes them, decode rows as
        ``prepare_decode_inputs`` does -- into one int64 buffer with one upload.  Returns input_ids /
        position_ids ``[1, C + D]`` and the metadata, all views of that buffer: the chunks' C tokens
        back to back (ragged rows, row b from token ``chunk_first[b]``), then the D decode tokens.
        With reference numerics (C, D) is ``padded_mixed_shape`` of the chunk tokens and the decode
        rows (pad tokens belong to no row, pad decode rows append nothing and attend to nothing),
        whether a graph replays the step or not; otherwise C is the chunk tokens and D the decode
        rows, unless a graph bucket pads them.  The metadata carries the live decode rows and the
        rows' first tokens on the host."""
        self._mixed_loaded = None
        live = len(decode_block_tables)
        lens = [len(c) for c in chunk_token_ids]
        width, total = max(lens), sum(lens)
        host = {"live_decode_rows": live, "chunk_first_host": tuple(int(x) for x in np.cumsum([0] + lens[:-1]))}
        exact = getattr(self.model, "exact", False)
        pad_chunk, pad_rows = padded_mixed_shape(total, live) if exact else (None, None)
        if self._mixed_graphs and pool is self._mixed_pool:
            hist = max(-(-st // pool.block_size) for st in start_positions)
            graph = self._mixed_bucket(len(chunk_token_ids), width, total, hist, live,
                                       max((len(t) for t in decode_block_tables), default=0))
            if graph is not None and exact and (graph.chunk_tokens, graph.decode_rows) != (pad_chunk, pad_rows):
                graph = None  # not this step's shape (the eager forward below runs it)
            if graph is not None:
                flat, _ = pack_mixed_rows(chunk_token_ids, start_positions, prefill_block_tables, last_tokens, positions,
                                          decode_block_tables, pool.block_size, self.pad_token_id,
                                          chunk_tokens=graph.chunk_tokens, history_blocks=graph.hist_blocks,
                                          decode_rows=graph.decode_rows, decode_blocks=graph.decode_blocks)
                graph.load(flat)
                self._mixed_loaded = (graph, live)
                ids, pos, meta = graph.views()
                return ids, pos, meta._replace(kv_pools=tuple(pool.kv_pools), **host)
        flat, (rows, chunk_tokens, nb, decode_rows, mb) = pack_mixed_rows(
            chunk_token_ids, start_positions, prefill_block_tables, last_tokens, positions, decode_block_tables,
            pool.block_size, self.pad_token_id, chunk_tokens=pad_chunk, decode_rows=pad_rows)
        packed = torch.from_numpy(flat).to(self.device)
        tokens = chunk_tokens + decode_rows
        at = 2 * tokens
        chunk = packed[at:at + rows * (3 + nb)].view(rows, 3 + nb)
        at += rows * (3 + nb)
        dec = packed[at:].view(decode_rows, 2 + mb)
        pools = tuple(pool.kv_pools)
        metadata = PagedMixedMetadata(
            prefill=PagedPrefillMetadata(history_block_tables=chunk[:, 3:], start_lens=chunk[:, 0],
                                         chunk_lens=chunk[:, 1], kv_pools=pools),
            decode=PagedAttentionMetadata(slot_mapping=dec[:, 0], block_tables=dec[:, 2:], context_lens=dec[:, 1],
                                          kv_pools=pools),
            prefill_rows=rows, prefill_width=width, kv_pools=pools, chunk_first=chunk[:, 2],
            chunk_tokens=chunk_tokens, **host)
        return packed[:tokens].view(1, tokens), packed[tokens:2 * tokens].view(1, tokens), metadata

    def run_mixed_step(self, input_ids: torch.Tensor, position_ids: torch.Tensor,
                       metadata: PagedMixedMetadata) -> MixedStepOutput:
        """One forward over the chunks and the decode tokens: the decode rows' K/V go into the pool,
        the chunks' K/V come back as ``prefill_cache``; greedy tokens of both (of the live decode
        rows only, ``metadata.live_decode_rows``).  Inputs that ``prepare_mixed_inputs`` loaded
        into a captured bucket replay its graph."""
        loaded = self._mixed_loaded
        if loaded is not None and metadata.decode.slot_mapping.data_ptr() == loaded[0].static_slots_ptr:
            graph, live = loaded
            with StepTimer(self.device) as timer:
                graph.graph.replay()
                next_token = argmax_rows(graph.logits)
            tokens = next_token.tolist()
            return MixedStepOutput(tokens[:graph.rows], tokens[graph.rows:graph.rows + live],
                                   self._ragged_cache(graph.presents, metadata), timer.elapsed_ms)
        with StepTimer(self.device) as timer:
            logits, present = self.model(input_ids, position_ids=position_ids, attn_metadata=metadata,
                                         last_logits_only=True)
            next_token, _ = greedy_sample(logits)
        tokens = next_token.squeeze(-1).tolist()
        rows = metadata.prefill_rows
        live = len(tokens) - rows if metadata.live_decode_rows is None else metadata.live_decode_rows
        cache = self._ragged_cache(present, metadata) if metadata.chunk_first is not None else KVCache(present)
        return MixedStepOutput(tokens[:rows], tokens[rows:rows + live], cache, timer.elapsed_ms)

    @staticmethod
    def _ragged_cache(present, metadata: PagedMixedMetadata) -> KVCache:
        """The chunk K/V of a ragged mixed step (one cached row of all chunk tokens), with the first
        token of each chunk row for ``store_prefill``: the metadata's host copy, else its device
        rows clamped as the attention kernels clamp them (to [0, C - len])."""
        cache = KVCache(present)
        first = metadata.chunk_first_host
        if first is None:
            lens = metadata.prefill.chunk_lens.clamp(0, metadata.prefill_width)
            first = tuple(torch.minimum(metadata.chunk_first.clamp(min=0), metadata.chunk_span - lens).tolist())
        cache.ragged_first = list(first)
        return cache


__all__ = ["MixedStepOutput", "PagedDecodeOutput", "PagedRunner"]
