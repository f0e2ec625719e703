"""Seeded synthetic inputs of the paged-KV workloads at Qwen3-0.6B attention shape.

Shapes: 16 query heads, 8 KV heads, head_dim 128, bf16, block_size 16, 28 layers.
Context lengths, block tables and values are all drawn from seeded generators, so the
GPU path and the CPU oracle see identical inputs:

* ``decode_step`` -- one layer: batch 8, contexts uniform in [64, 512], pool 4096 blocks,
  block tables from one random permutation of blocks 1..4095.
* ``prefill_scatter`` -- 28 layers: 32 prompts, lengths uniform in [128, 2048], block tables
  from ``FreeKVCacheBlockQueue`` after seeded churn: ``fragmented`` (decode-style interleaved
  growth; under 1% of neighbouring entries consecutive) or ``near_sequential`` (a short churn at
  the front of the pool; about 99% consecutive).
* ``decode_at_scale`` -- 28 layers: batch 256, contexts lognormal (median 2048, sigma 1.3,
  clipped to [256, 8192]; about 90 GB of K/V), randomly permuted blocks.
* ``chunked_prefill`` -- 4 prompts of 16384 tokens in 2048-token chunks with history, tables of
  either kind.
* ``serving_requests`` -- the continuous-batching run: 128 requests, Poisson arrivals at 20 req/s
  (exponential gaps, mean 50 ms, first arrival at 0), prompt lengths uniform in [32, 1024] with
  token ids uniform in [1000, 100000), 128 output tokens each.

Small values (context counts, tables) are drawn on the CPU with ``torch.Generator``; bulk
values are drawn with ``randn`` in fp32 and cast to bf16, on the CPU for the small workloads
and on the GPU (seeded CUDA generator) for the ~90 GB pool.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from mini_infra_qwen3_amd.core.block_manager import FreeKVCacheBlockQueue, num_blocks_for_tokens

NUM_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
BLOCK_SIZE = 16
NUM_LAYERS = 28
SCALE = HEAD_DIM ** -0.5
KV_BYTES_PER_TOKEN_LAYER = 2 * NUM_KV_HEADS * HEAD_DIM * 2  # K + V, bf16: 4096 B


def _randn_bf16(shape, gen: torch.Generator, device: torch.device | str = "cpu") -> torch.Tensor:
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)


def uniform_lengths(n: int, lo: int, hi: int, gen: torch.Generator) -> list[int]:
    return torch.randint(lo, hi + 1, (n,), generator=gen).tolist()


def lognormal_lengths(n: int, median: float, sigma: float, lo: int, hi: int, gen: torch.Generator) -> list[int]:
    z = torch.randn(n, generator=gen, dtype=torch.float64)
    return torch.exp(math.log(median) + sigma * z).round().clamp(lo, hi).long().tolist()


def permuted_tables(lengths: list[int], num_blocks: int, gen: torch.Generator,
                    block_size: int = BLOCK_SIZE) -> list[list[int]]:
    """Splits one random permutation of blocks 1..num_blocks-1 into per-sequence tables."""
    need = [num_blocks_for_tokens(n, block_size) for n in lengths]
    if sum(need) > num_blocks - 1:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {sum(need)} blocks")
    perm = (torch.randperm(num_blocks - 1, generator=gen) + 1).tolist()
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n])
        k += n
    return tables


def churned_tables(lengths: list[int], num_blocks: int, gen: torch.Generator, block_size: int = BLOCK_SIZE,
                   churn_rounds: int = 64) -> list[list[int]]:
    """Near-sequential tables: a FreeKVCacheBlockQueue after a short seeded alloc/free churn of 64
    dummy requests, all freed again before the measured allocation.  The churn touches only the front
    of the pool, so the allocation then runs mostly over never-used blocks: about 99% of adjacent
    table entries are consecutive block ids."""
    queue = FreeKVCacheBlockQueue(num_blocks)
    live: list[list[int]] = []
    for _ in range(churn_rounds):
        if live and torch.rand(1, generator=gen).item() < 0.45:
            victim = int(torch.randint(len(live), (1,), generator=gen))
            queue.free(live.pop(victim))
        else:
            n = int(torch.randint(1, 48, (1,), generator=gen))
            if n <= queue.num_free_blocks:
                live.append(queue.allocate(n))
    for blocks in live:
        queue.free(blocks)
    return [queue.allocate(num_blocks_for_tokens(n, block_size)) for n in lengths]


def fragmented_tables(lengths: list[int], num_blocks: int, gen: torch.Generator, block_size: int = BLOCK_SIZE,
                      streams: int = 64) -> list[list[int]]:
    """Tables from a FreeKVCacheBlockQueue whose free list was reordered the way decoding reorders it:
    ``streams`` requests each take one block per round, in a fresh random order every round, until
    the pool is used up; they then finish in a random order and free their blocks.  The free list
    then interleaves the requests' blocks, so a new table's neighbouring entries are almost never
    consecutive block ids (under 1% at the default 64 streams) and each 32 KiB block of one layer's
    K or V lies at its own place in the pool."""
    queue = FreeKVCacheBlockQueue(num_blocks)
    held: list[list[int]] = [[] for _ in range(streams)]
    while queue.num_free_blocks:
        for s in torch.randperm(streams, generator=gen).tolist():
            if not queue.num_free_blocks:
                break
            held[s].extend(queue.allocate(1))
    for s in torch.randperm(streams, generator=gen).tolist():
        queue.free(held[s])
    return [queue.allocate(num_blocks_for_tokens(n, block_size)) for n in lengths]


TABLE_KINDS = {"fragmented": fragmented_tables, "near_sequential": churned_tables}


def consecutive_fraction(tables: list[list[int]]) -> float:
    """Fraction of adjacent table entries that are consecutive block ids (next == previous + 1)."""
    pairs = sum(max(len(t) - 1, 0) for t in tables)
    if pairs == 0:
        return 0.0
    hits = sum(int(np.count_nonzero(np.diff(np.asarray(t, dtype=np.int64)) == 1)) for t in tables if len(t) > 1)
    return hits / pairs


def padded(tables: list[list[int]]) -> torch.Tensor:
    width = max(len(t) for t in tables)
    out = torch.zeros((len(tables), width), dtype=torch.long)
    for b, t in enumerate(tables):
        out[b, :len(t)] = torch.tensor(t, dtype=torch.long)
    return out


def slots_of(tables: list[list[int]], positions: list[int], block_size: int = BLOCK_SIZE) -> torch.Tensor:
    return torch.tensor([t[p // block_size] * block_size + p % block_size for t, p in zip(tables, positions)],
                        dtype=torch.long)


@dataclass
class DecodeWorkload:
    """Inputs of paged decode steps (CPU tensors unless noted)."""

    context_lens: list[int]          # includes the new token
    tables: list[list[int]]
    block_tables: torch.Tensor       # [B, max_blocks] null-padded
    num_blocks: int
    num_layers: int
    query: torch.Tensor              # [L, B, H, D] (device)
    new_key: torch.Tensor            # [L, B, Hkv, D] (device)
    new_value: torch.Tensor          # [L, B, Hkv, D] (device)
    pools: torch.Tensor              # [L, 2, num_blocks, bs, Hkv, D] (device)

    @property
    def slot_mapping(self) -> torch.Tensor:
        return slots_of(self.tables, [n - 1 for n in self.context_lens])

    @property
    def kv_bytes_per_layer(self) -> int:
        """Algorithmic K+V bytes one decode-attention layer reads: sum of contexts x 4096 B."""
        return sum(self.context_lens) * KV_BYTES_PER_TOKEN_LAYER


def decode_step(seed: int = 0, device: torch.device | str = "cpu", batch: int = 8, num_blocks: int = 4096,
                lo: int = 64, hi: int = 512) -> DecodeWorkload:
    """One paged decode layer: contexts U[lo, hi], pool ``num_blocks``, permuted tables, values CPU-drawn."""
    gen = torch.Generator().manual_seed(seed)
    ctx = uniform_lengths(batch, lo, hi, gen)
    tables = permuted_tables(ctx, num_blocks, gen)
    pools = _randn_bf16((1, 2, num_blocks, BLOCK_SIZE, NUM_KV_HEADS, HEAD_DIM), gen)
    query = _randn_bf16((1, batch, NUM_HEADS, HEAD_DIM), gen)
    new_k = _randn_bf16((1, batch, NUM_KV_HEADS, HEAD_DIM), gen)
    new_v = _randn_bf16((1, batch, NUM_KV_HEADS, HEAD_DIM), gen)
    return DecodeWorkload(ctx, tables, padded(tables), num_blocks, 1, query.to(device), new_k.to(device),
                          new_v.to(device), pools.to(device))


def decode_at_scale(seed: int = 0, device: torch.device | str = "cuda", batch: int = 256,
                    num_layers: int = NUM_LAYERS, median: float = 2048.0, sigma: float = 1.3,
                    lo: int = 256, hi: int = 8192) -> DecodeWorkload:
    """Decode at scale: lognormal contexts, pool sized to hold them all, bulk values drawn on ``device``."""
    gen = torch.Generator().manual_seed(seed)
    ctx = lognormal_lengths(batch, median, sigma, lo, hi, gen)
    num_blocks = 1 + sum(num_blocks_for_tokens(n, BLOCK_SIZE) for n in ctx)
    tables = permuted_tables(ctx, num_blocks, gen)
    dgen = torch.Generator(device=device).manual_seed(seed + 1)
    pools = torch.empty((num_layers, 2, num_blocks, BLOCK_SIZE, NUM_KV_HEADS, HEAD_DIM), dtype=torch.bfloat16,
                        device=device)
    for layer in range(num_layers):  # layer by layer keeps the fp32 temporary small
        for kv in range(2):
            pools[layer, kv].copy_(torch.randn(pools.shape[2:], generator=dgen, device=device))
    query = _randn_bf16((num_layers, batch, NUM_HEADS, HEAD_DIM), dgen, device)
    new_k = _randn_bf16((num_layers, batch, NUM_KV_HEADS, HEAD_DIM), dgen, device)
    new_v = _randn_bf16((num_layers, batch, NUM_KV_HEADS, HEAD_DIM), dgen, device)
    return DecodeWorkload(ctx, tables, padded(tables), num_blocks, num_layers, query, new_k, new_v, pools)


@dataclass
class PrefillScatterWorkload:
    """Inputs of a multi-layer prefill scatter."""

    lengths: list[int]
    tables: list[list[int]]
    num_blocks: int
    padded_length: int
    sources: torch.Tensor            # [L, 2, B, Hkv, padded_length, D] (device); left-padded prompts
    index: np.ndarray                # [3, N] token_rows, token_positions, slots

    @property
    def num_tokens(self) -> int:
        return int(sum(self.lengths))


def prefill_scatter(seed: int = 0, device: torch.device | str = "cuda", num_prompts: int = 32,
                    lo: int = 128, hi: int = 2048, num_layers: int = NUM_LAYERS,
                    num_blocks: int | None = None, tables: str = "fragmented") -> PrefillScatterWorkload:
    """Whole-prompt prefill scatter: prompts U[lo, hi], tables of kind ``tables`` (a key of
    ``TABLE_KINDS``), sources drawn on ``device``."""
    from mini_infra_qwen3_amd.worker.metadata import prefill_scatter_indices

    gen = torch.Generator().manual_seed(seed)
    lengths = uniform_lengths(num_prompts, lo, hi, gen)
    need = sum(num_blocks_for_tokens(n, BLOCK_SIZE) for n in lengths)
    num_blocks = num_blocks or 1 + need + 512
    tables = TABLE_KINDS[tables](lengths, num_blocks, gen)
    width = max(lengths)
    dgen = torch.Generator(device=device).manual_seed(seed + 1)
    sources = _randn_bf16((num_layers, 2, num_prompts, NUM_KV_HEADS, width, HEAD_DIM), dgen, device)
    index = prefill_scatter_indices(tables, lengths, [0] * num_prompts, width, BLOCK_SIZE)
    return PrefillScatterWorkload(lengths, tables, num_blocks, width, sources, index)


@dataclass
class ChunkedPrefillWorkload:
    """A long prompt processed in fixed-size chunks: per prompt block table and all Q/K/V."""

    prompt_len: int
    chunk_len: int
    num_prompts: int
    tables: list[list[int]]
    num_blocks: int

    @property
    def num_chunks(self) -> int:
        return self.prompt_len // self.chunk_len

    def history_bytes_per_layer(self) -> int:
        """K+V bytes the history reads of all chunks take, per layer: sum over chunks of start x 4096 B."""
        starts = [c * self.chunk_len for c in range(self.num_chunks)]
        return self.num_prompts * sum(starts) * KV_BYTES_PER_TOKEN_LAYER


def chunked_prefill(seed: int = 0, num_prompts: int = 4, prompt_len: int = 16384,
                    chunk_len: int = 2048, tables: str = "fragmented") -> ChunkedPrefillWorkload:
    """Long prompts in fixed-size chunks; block tables of kind ``tables`` (a key of ``TABLE_KINDS``)."""
    gen = torch.Generator().manual_seed(seed)
    num_blocks = 1 + num_prompts * num_blocks_for_tokens(prompt_len, BLOCK_SIZE) + 256
    tables = TABLE_KINDS[tables]([prompt_len] * num_prompts, num_blocks, gen)
    return ChunkedPrefillWorkload(prompt_len, chunk_len, num_prompts, tables, num_blocks)


def serving_requests(seed: int = 0, num_requests: int = 128, rate_per_s: float = 20.0, min_prompt: int = 32,
                     max_prompt: int = 1024, max_new_tokens: int = 128, vocab_size: int = 151936):
    """Requests of the continuous-batching run (pure Poisson arrivals: no initial burst, no clamping
    of the gaps).  Token ids span [1000, min(vocab, 100000)) as the reference's synthetic prompts do
    (src/mini_infra/bench/synthetic.py:29-31)."""
    from mini_infra_qwen3_amd.core.types import Request

    rng = np.random.default_rng(seed)
    gaps = rng.exponential(1000.0 / rate_per_s, num_requests)
    gaps[0] = 0.0
    arrivals = np.round(np.cumsum(gaps), 3)
    lengths = rng.integers(min_prompt, max_prompt + 1, num_requests)
    low = 1000 if vocab_size > 1000 else 1
    high = min(vocab_size, 100000)
    return [Request(i, tuple(int(t) for t in rng.integers(low, high, int(n))), max_new_tokens, float(a))
            for i, (n, a) in enumerate(zip(lengths, arrivals))]


__all__ = [
    "BLOCK_SIZE", "HEAD_DIM", "KV_BYTES_PER_TOKEN_LAYER", "NUM_HEADS", "NUM_KV_HEADS", "NUM_LAYERS", "SCALE",
    "TABLE_KINDS", "ChunkedPrefillWorkload", "DecodeWorkload", "PrefillScatterWorkload", "chunked_prefill",
    "churned_tables", "consecutive_fraction", "fragmented_tables",
    "decode_at_scale", "decode_step", "lognormal_lengths", "padded", "permuted_tables", "prefill_scatter",
    "serving_requests", "slots_of", "uniform_lengths",
]
