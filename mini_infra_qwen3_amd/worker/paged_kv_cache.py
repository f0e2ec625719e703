"""Physical block pool of the paged KV cache on one MI355X.

Same API and tensor layout as the reference's PagedKVCachePool
(src/mini_infra/worker/paged_kv_cache.py:14-95): ``kv_pools[layer] = (key_pool, value_pool)``,
each ``[num_blocks, block_size, num_kv_heads, head_dim]``, zero-filled, block 0 the null block,
``slot = block_id * block_size + offset``.

MI355X layout: all layers live in ONE allocation ``[num_layers, 2, num_blocks, bs, H, D]`` (a
90 GB pool is a single HBM3E range), and ``kv_pools`` are views of it, so the per-layer tensors
the reference's callers index are unchanged.  ``gather_blocks`` and ``write_prefill`` are single
HIP launches over all layers (kernels 2 and 1) instead of per-layer advanced indexing.
"""

from __future__ import annotations

import math

import torch

from mini_infra_qwen3_amd import data_plane
from mini_infra_qwen3_amd.worker.kv_cache import KVCache


class PagedKVCachePool:
    """Per-layer physical K/V block pools, GPU only (there is no CPU data plane)."""

    def __init__(
        self,
        num_layers: int,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str,
    ):
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError(f"PagedKVCachePool needs a GPU device, got {device} (no CPU data plane)")
        if num_layers < 1 or num_blocks < 1 or block_size < 1 or num_kv_heads < 1 or head_dim < 1:
            raise ValueError("PagedKVCachePool: every dimension must be positive")
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.storage = torch.zeros(
            (num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim), dtype=dtype, device=device
        )
        self.kv_pools: list[tuple[torch.Tensor, torch.Tensor]] = [
            (self.storage[layer, 0], self.storage[layer, 1]) for layer in range(num_layers)
        ]

    @property
    def device(self) -> torch.device:
        return self.storage.device

    @property
    def bytes_per_block(self) -> int:
        """K+V bytes of one physical block across all layers."""
        key_pool, _ = self.kv_pools[0]
        return 2 * len(self.kv_pools) * math.prod(key_pool.shape[1:]) * key_pool.element_size()

    @property
    def total_bytes(self) -> int:
        """Bytes of the whole pool, null block included."""
        return self.num_blocks * self.bytes_per_block

    def gather_blocks(self, block_ids: torch.Tensor) -> tuple[tuple[torch.Tensor, torch.Tensor], ...]:
        """History K/V by block table, every layer in one kernel launch.

        block_ids: ``[B, nb]`` int64 on the pool's device, right-padded with the null block.
        Returns per layer ``(key, value)``, each ``[B, H_kv, nb * block_size, D]`` -- non-contiguous
        ``transpose(1, 2)`` views of a contiguous ``[B, nb * block_size, H_kv, D]`` gather, exactly
        as the reference returns them (whole blocks, null block and stale tails included).
        """
        if block_ids.ndim != 2:
            raise ValueError(f"block_ids must be [batch, num_blocks], got {tuple(block_ids.shape)}")
        block_ids = block_ids.to(device=self.device, dtype=torch.long)
        batch, nb = block_ids.shape
        num_layers = len(self.kv_pools)
        out = torch.empty(
            (num_layers, 2, batch, nb * self.block_size, self.num_kv_heads, self.head_dim),
            dtype=self.storage.dtype, device=self.device,
        )
        keys = [out[layer, 0] for layer in range(num_layers)]
        values = [out[layer, 1] for layer in range(num_layers)]
        data_plane.gather_blocks(
            [k for k, _ in self.kv_pools], [v for _, v in self.kv_pools], block_ids, keys, values
        )
        return tuple((k.transpose(1, 2), v.transpose(1, 2)) for k, v in zip(keys, values))

    def _block_id_tensor(self, block_ids, unique: bool) -> torch.Tensor:
        if isinstance(block_ids, torch.Tensor):
            return block_ids.to(device=self.device, dtype=torch.long).reshape(-1)
        ids = [int(b) for b in block_ids]
        if any(not 0 <= b < self.num_blocks for b in ids):
            raise ValueError(f"block ids must lie in [0, {self.num_blocks})")
        if unique and len(set(ids)) != len(ids):
            raise ValueError("block ids written by one call must be unique")
        return torch.tensor(ids, dtype=torch.long).to(self.device, non_blocking=True)

    def pack_blocks(self, block_ids) -> torch.Tensor:
        """Blocks ``block_ids`` of every layer as contiguous KV block records
        ``[n, num_layers, 2, bs, H, D]`` (the swap / wire format), one kernel launch."""
        return data_plane.pack_blocks([k for k, _ in self.kv_pools], [v for _, v in self.kv_pools],
                                      self._block_id_tensor(block_ids, unique=False))

    def unpack_blocks(self, records: torch.Tensor, block_ids) -> None:
        """Writes KV block records into blocks ``block_ids`` (unique) of every layer, one kernel launch."""
        data_plane.unpack_blocks(records, [k for k, _ in self.kv_pools], [v for _, v in self.kv_pools],
                                 self._block_id_tensor(block_ids, unique=True))

    def write_prefill(
        self,
        prefill_cache: KVCache,
        token_rows: torch.Tensor,
        token_positions: torch.Tensor,
        slot_mapping: torch.Tensor,
    ) -> None:
        """Scatters the valid prefill tokens of every layer into their slots (one kernel launch).

        prefill_cache: per layer ``(key, value)``, each ``[B, H_kv, L, D]`` (any strides, D contiguous).
        token_rows / token_positions / slot_mapping: ``[N]`` int64; slots must be unique.
        """
        caches = list(prefill_cache)
        if len(caches) != len(self.kv_pools):
            raise ValueError(f"prefill_cache has {len(caches)} layers, pool has {len(self.kv_pools)}")
        data_plane.reshape_and_cache(
            [k for k, _ in caches],
            [v for _, v in caches],
            slot_mapping,
            [k for k, _ in self.kv_pools],
            [v for _, v in self.kv_pools],
            token_rows=token_rows,
            token_positions=token_positions,
        )


__all__ = ["PagedKVCachePool"]
