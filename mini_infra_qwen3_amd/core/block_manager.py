"""Logical block allocator of the paged KV cache: FIFO free-block queue and per-request block tables.

The reference's API and observable behaviour (src/mini_infra/core/block_manager.py:17-149): block
ids 1..num_blocks-1 handed out first-freed-first-reused (block 0 is the null block that pads
tables), the cold / reuse / release / peak counters, all-or-nothing slot allocation and FCFS
admission under a reservation.  The state behind it is a few preallocated int64 arrays instead
of Python containers:

* The free queue is a ring over an array holding every allocatable id once.  ``allocate`` takes
  a slice at the head and ``free`` writes at the tail.  The queue starts as 1, 2, ..., n - 1 and
  freed ids always queue behind the never-used ones, so the first n - 1 ids ever handed out are
  exactly the cold allocations and every later one is a reuse: two counters replace a set of
  every id ever allocated.
* Block tables are the rows of one int64 matrix, grown by doubling, null-padded.  A request owns
  a row for its lifetime; freed rows are reused.  Every entry ``allocate_slots`` writes is also
  logged as a ``(row, column, block id)`` delta, so a device copy of the matrix
  (``worker.block_tables.DeviceBlockTables``) stays current by uploading the deltas alone:
  one id per request whenever a decode step crosses a block boundary, instead of re-packing
  every table every step.
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence

import numpy as np

NULL_BLOCK_ID = 0


def num_blocks_for_tokens(num_tokens: int, block_size: int) -> int:
    """Blocks needed to hold ``num_tokens`` tokens (ceil). Reference block_manager.py:20-22."""
    return -(-num_tokens // block_size)


def required_pool_blocks(requests: Iterable, max_running_requests: int, block_size: int) -> int:
    """Pool size (null block included) that no ``max_running_requests`` concurrent requests can exhaust.

    A request holds at most ``prompt_len + max_new_tokens - 1`` tokens (its last generated token is
    never fed back), so the bound is the blocks of the largest ``max_running_requests`` of those.
    Reference block_manager.py:25-32.
    """
    peaks = np.sort(np.fromiter((r.prompt_len + r.max_new_tokens - 1 for r in requests), dtype=np.int64))[::-1]
    top = peaks[:max_running_requests]
    return 1 + int(np.sum(-(-top // block_size)))


class FreeKVCacheBlockQueue:
    """FIFO queue of the free physical block ids 1..num_blocks-1 on a ring buffer.

    Reference block_manager.py:35-76: ``allocate(n)`` returns the n oldest free ids (RuntimeError
    when fewer are free), ``free(ids)`` queues ids behind the rest; counters ``num_free_blocks``,
    ``num_used_blocks`` (null block excluded), ``peak_used_blocks``, ``block_cold_allocation_count``
    (first allocations of an id), ``reuse_count`` and ``release_count``.  Only ids this queue handed
    out may be freed, once each (as the reference assumes); freeing more ids than are allocated
    raises RuntimeError instead of corrupting the queue.
    """

    def __init__(self, num_blocks: int):
        if num_blocks < 2:
            raise ValueError("num_blocks must be at least 2 (block 0 is the null block)")
        self.num_blocks = num_blocks
        self._ring = np.arange(NULL_BLOCK_ID + 1, num_blocks, dtype=np.int64)
        self._head = 0            # ring position of the oldest free id
        self._count = num_blocks - 1
        self._handed_out = 0      # ids ever handed out
        self.release_count = 0
        self.peak_used_blocks = 0

    @property
    def num_free_blocks(self) -> int:
        return self._count

    @property
    def num_used_blocks(self) -> int:
        """Allocated blocks, null block excluded."""
        return self.num_blocks - 1 - self._count

    @property
    def block_cold_allocation_count(self) -> int:
        return min(self._handed_out, self._ring.shape[0])

    @property
    def reuse_count(self) -> int:
        return self._handed_out - self.block_cold_allocation_count

    def allocate(self, num_blocks: int) -> list[int]:
        """The ``num_blocks`` oldest free ids, in queue order."""
        if num_blocks > self._count:
            raise RuntimeError(f"not enough free blocks: need {num_blocks}, have {self._count}")
        cap = self._ring.shape[0]
        start, end = self._head, self._head + num_blocks
        if end <= cap:
            taken = self._ring[start:end].tolist()
        else:
            taken = self._ring[start:].tolist() + self._ring[:end - cap].tolist()
        self._head = end % cap if cap else 0
        self._count -= num_blocks
        self._handed_out += num_blocks
        self.peak_used_blocks = max(self.peak_used_blocks, self.num_used_blocks)
        return taken

    def free(self, block_ids: Sequence[int]) -> None:
        """Queues ids behind every free one (freed blocks keep their stale contents)."""
        ids = np.asarray(block_ids, dtype=np.int64).reshape(-1)
        n = ids.shape[0]
        cap = self._ring.shape[0]
        if self._count + n > cap:
            raise RuntimeError(f"freeing {n} blocks with only {cap - self._count} allocated")
        tail = (self._head + self._count) % cap
        first = min(n, cap - tail)
        self._ring[tail:tail + first] = ids[:first]
        self._ring[:n - first] = ids[first:]
        self._count += n
        self.release_count += n


class KVCacheManager:
    """Per-request block tables grown block by block. Reference block_manager.py:79-149.

    ``block_table(idx)`` returns a request's table as a list (logical block -> physical id); the
    same tables are the rows of ``table_matrix`` (``row_of(idx)``), and ``take_deltas()`` hands out
    the entries written since the previous call.
    """

    def __init__(self, block_size: int, num_blocks: int):
        if block_size < 1:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self.free_block_queue = FreeKVCacheBlockQueue(num_blocks)
        self._row_of: dict[int, int] = {}
        self._spare_rows: list[int] = []
        self._matrix = np.zeros((8, 8), dtype=np.int64)   # rows x blocks, null-padded
        self._blocks = np.zeros(8, dtype=np.int64)         # blocks per row
        self._tokens = np.zeros(8, dtype=np.int64)         # tokens per row
        self._rows_used = 0
        self._delta_rows: list[np.ndarray] = []
        self._delta_cols: list[np.ndarray] = []
        self._delta_ids: list[np.ndarray] = []

    # -- counters (reference block_manager.py:97-115) -----------------------------------------
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

    # -- tables --------------------------------------------------------------------------------
    def block_table(self, request_idx: int) -> list[int]:
        """Logical block index -> physical block id of one request (KeyError if unknown)."""
        row = self._row_of[request_idx]
        return self._matrix[row, :self._blocks[row]].tolist()

    def row_of(self, request_idx: int) -> int:
        """The table-matrix row of a live request (KeyError if unknown)."""
        return self._row_of[request_idx]

    @property
    def table_matrix(self) -> np.ndarray:
        """``[rows, width]`` int64: row r holds its request's table, then stale ids or the null block."""
        return self._matrix

    def num_tokens(self, request_idx: int) -> int:
        return int(self._tokens[self._row_of[request_idx]])

    def take_deltas(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """(rows, columns, ids) of every table entry written since the last call."""
        if not self._delta_rows:
            empty = np.zeros(0, dtype=np.int64)
            return empty, empty, empty
        out = (np.concatenate(self._delta_rows), np.concatenate(self._delta_cols), np.concatenate(self._delta_ids))
        self._delta_rows, self._delta_cols, self._delta_ids = [], [], []
        return out

    def _new_row(self) -> int:
        if self._spare_rows:
            return self._spare_rows.pop()
        row = self._rows_used
        if row == self._matrix.shape[0]:
            grown = self._matrix.shape[0] * 2
            self._matrix = np.pad(self._matrix, ((0, grown - self._matrix.shape[0]), (0, 0)))
            self._blocks = np.pad(self._blocks, (0, grown - self._blocks.shape[0]))
            self._tokens = np.pad(self._tokens, (0, grown - self._tokens.shape[0]))
        self._rows_used += 1
        return row

    # -- admission and allocation (reference block_manager.py:117-149) ----------------------
    def num_admissible(self, prompt_lens: Sequence[int], num_reserved_blocks: int) -> int:
        """How many requests, in FCFS order, fit into the free blocks left after the reservation:
        the longest prefix whose block needs add up to at most that budget."""
        budget = self.free_block_queue.num_free_blocks - num_reserved_blocks
        need = -(-np.asarray(prompt_lens, dtype=np.int64) // self.block_size)
        return int(np.searchsorted(np.cumsum(need), budget, side="right"))

    def allocate_slots(self, request_idx: int, num_new_tokens: int) -> bool:
        """Adds room for ``num_new_tokens`` tokens; all-or-nothing (False leaves no trace)."""
        row = self._row_of.get(request_idx)
        have_blocks = int(self._blocks[row]) if row is not None else 0
        total = (int(self._tokens[row]) if row is not None else 0) + num_new_tokens
        extra = num_blocks_for_tokens(total, self.block_size) - have_blocks
        if extra > self.free_block_queue.num_free_blocks:
            return False
        if row is None:
            row = self._new_row()
            self._row_of[request_idx] = row
        if extra > 0:
            ids = np.asarray(self.free_block_queue.allocate(extra), dtype=np.int64)
            end = have_blocks + extra
            if end > self._matrix.shape[1]:
                width = max(end, 2 * self._matrix.shape[1])
                self._matrix = np.pad(self._matrix, ((0, 0), (0, width - self._matrix.shape[1])))
            self._matrix[row, have_blocks:end] = ids
            self._blocks[row] = end
            self._delta_rows.append(np.full(extra, row, dtype=np.int64))
            self._delta_cols.append(np.arange(have_blocks, end, dtype=np.int64))
            self._delta_ids.append(ids)
        self._tokens[row] = total
        return True

    def free(self, request_idx: int) -> None:
        """Returns every block of the request to the free queue and its row to the spare rows."""
        row = self._row_of.pop(request_idx)
        n = int(self._blocks[row])
        self.free_block_queue.free(self._matrix[row, :n].copy())
        self._blocks[row] = 0
        self._tokens[row] = 0
        self._spare_rows.append(row)


__all__ = [
    "FreeKVCacheBlockQueue",
    "KVCacheManager",
    "NULL_BLOCK_ID",
    "num_blocks_for_tokens",
    "required_pool_blocks",
]
