"""CPU restatement of the reference's block allocator (oracle; test infrastructure only).

Follows src/mini_infra/core/block_manager.py:35-149 with the reference's own containers (a deque
of free ids, a set of ids ever handed out, a list per request), so that the array-backed
allocator of the product can be checked against it operation by operation.
"""

from __future__ import annotations

from collections import deque


class ReferenceBlockAllocator:
    """FreeKVCacheBlockQueue + KVCacheManager of the reference (block_manager.py:35-149)."""

    def __init__(self, block_size: int, num_blocks: int):
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.free_ids = deque(range(1, num_blocks))
        self.ever = set()
        self.cold = self.reuse = self.release = self.peak = 0
        self.tables: dict[int, list[int]] = {}
        self.tokens: dict[int, int] = {}

    @property
    def used(self) -> int:
        return self.num_blocks - 1 - len(self.free_ids)

    def _take(self, n: int) -> list[int]:
        if n > len(self.free_ids):
            raise RuntimeError("not enough free blocks")
        out = []
        for _ in range(n):
            b = self.free_ids.popleft()
            if b in self.ever:
                self.reuse += 1
            else:
                self.ever.add(b)
                self.cold += 1
            out.append(b)
        self.peak = max(self.peak, self.used)
        return out

    def num_admissible(self, prompt_lens, reserved: int) -> int:
        budget = len(self.free_ids) - reserved
        count = 0
        for n in prompt_lens:
            need = -(-n // self.block_size)
            if need > budget:
                break
            budget -= need
            count += 1
        return count

    def allocate_slots(self, idx: int, n: int) -> bool:
        table = self.tables.get(idx, [])
        total = self.tokens.get(idx, 0) + n
        extra = -(-total // self.block_size) - len(table)
        if extra > len(self.free_ids):
            return False
        table.extend(self._take(extra))
        self.tables[idx] = table
        self.tokens[idx] = total
        return True

    def free(self, idx: int) -> None:
        ids = self.tables.pop(idx)
        del self.tokens[idx]
        self.free_ids.extend(ids)
        self.release += len(ids)
