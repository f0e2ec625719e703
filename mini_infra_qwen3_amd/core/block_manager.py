"""Logical block allocator of the paged KV cache: FIFO free-block queue and per-request block tables.

Pure CPU control plane with the reference's API and behaviour
(src/mini_infra/core/block_manager.py:17-149): it hands out integer physical block ids and
never touches device memory.  Block 0 is the null block: never allocated, used to right-pad
block tables so padded entries still address valid pool memory.
"""

from __future__ import annotations

from collections import deque
from collections.abc import Iterable, Sequence

NULL_BLOCK_ID = 0


def num_blocks_for_tokens(num_tokens: int, block_size: int) -> int:
    """Blocks needed to hold ``num_tokens`` tokens (ceil). Reference block_manager.py:20-22."""
    return -(-num_tokens // block_size)


def required_pool_blocks(requests: Iterable, max_running_requests: int, block_size: int) -> int:
    """Pool size (null block included) that no ``max_running_requests`` concurrent requests can exhaust.

    A request holds at most ``prompt_len + max_new_tokens - 1`` tokens (the last generated token
    is never fed back); the bound sums the largest ``max_running_requests`` of those.
    Reference block_manager.py:25-32.
    """
    peaks = sorted((r.prompt_len + r.max_new_tokens - 1 for r in requests), reverse=True)
    return 1 + sum(num_blocks_for_tokens(t, block_size) for t in peaks[:max_running_requests])


class FreeKVCacheBlockQueue:
    """FIFO queue of free physical block ids 1..num_blocks-1 (first freed, first reused).

    Reference block_manager.py:35-76, including the cold/reuse/release/peak counters.
    """

    def __init__(self, num_blocks: int):
        if num_blocks < 2:
            raise ValueError("num_blocks must be at least 2 (block 0 is the null block)")
        self.num_blocks = num_blocks
        self._free: deque[int] = deque(range(NULL_BLOCK_ID + 1, num_blocks))
        self._seen: set[int] = set()
        self.block_cold_allocation_count = 0
        self.reuse_count = 0
        self.release_count = 0
        self.peak_used_blocks = 0

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    @property
    def num_used_blocks(self) -> int:
        """Allocated blocks, null block excluded."""
        return self.num_blocks - 1 - len(self._free)

    def allocate(self, num_blocks: int) -> list[int]:
        """Pops ``num_blocks`` ids from the front; RuntimeError if not enough are free."""
        if num_blocks > len(self._free):
            raise RuntimeError(f"not enough free blocks: need {num_blocks}, have {len(self._free)}")
        taken = [self._free.popleft() for _ in range(num_blocks)]
        for block_id in taken:
            if block_id in self._seen:
                self.reuse_count += 1
            else:
                self._seen.add(block_id)
                self.block_cold_allocation_count += 1
        self.peak_used_blocks = max(self.peak_used_blocks, self.num_used_blocks)
        return taken

    def free(self, block_ids: Sequence[int]) -> None:
        """Appends ids to the back of the queue (freed blocks keep their stale contents)."""
        self._free.extend(block_ids)
        self.release_count += len(block_ids)


class KVCacheManager:
    """Per-request block tables grown block by block. Reference block_manager.py:79-149."""

    def __init__(self, block_size: int, num_blocks: int):
        if block_size < 1:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self.free_block_queue = FreeKVCacheBlockQueue(num_blocks)
        self._tables: dict[int, list[int]] = {}
        self._tokens: dict[int, int] = {}

    @property
    def num_used_blocks(self) -> int:
        return self.free_block_queue.num_used_blocks

    @property
    def block_cold_allocation_count(self) -> int:
        return self.free_block_queue.block_cold_allocation_count

    @property
    def block_reuse_count(self) -> int:
        return self.free_block_queue.reuse_count

    @property
    def block_release_count(self) -> int:
        return self.free_block_queue.release_count

    @property
    def peak_used_blocks(self) -> int:
        return self.free_block_queue.peak_used_blocks

    def block_table(self, request_idx: int) -> list[int]:
        """Logical block index -> physical block id of one request (KeyError if unknown)."""
        return self._tables[request_idx]

    def num_admissible(self, prompt_lens: Sequence[int], num_reserved_blocks: int) -> int:
        """How many requests, in FCFS order, fit into the free blocks left after the reservation."""
        budget = self.free_block_queue.num_free_blocks - num_reserved_blocks
        count = 0
        for prompt_len in prompt_lens:
            need = num_blocks_for_tokens(prompt_len, self.block_size)
            if need > budget:
                break
            budget -= need
            count += 1
        return count

    def allocate_slots(self, request_idx: int, num_new_tokens: int) -> bool:
        """Adds room for ``num_new_tokens`` tokens; all-or-nothing (False leaves no trace)."""
        table = self._tables.get(request_idx, [])
        total = self._tokens.get(request_idx, 0) + num_new_tokens
        extra = num_blocks_for_tokens(total, self.block_size) - len(table)
        if extra > self.free_block_queue.num_free_blocks:
            return False
        table.extend(self.free_block_queue.allocate(extra))
        self._tables[request_idx] = table
        self._tokens[request_idx] = total
        return True

    def free(self, request_idx: int) -> None:
        """Returns every block of the request to the free queue."""
        self.free_block_queue.free(self._tables.pop(request_idx))
        del self._tokens[request_idx]


__all__ = [
    "FreeKVCacheBlockQueue",
    "KVCacheManager",
    "NULL_BLOCK_ID",
    "num_blocks_for_tokens",
    "required_pool_blocks",
]
