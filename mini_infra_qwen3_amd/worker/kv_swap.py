"""KV block records: swapping physical KV blocks to a pinned host pool, and a file format for them.

The reference plans a "swap" preemption mode: a victim's physical KV blocks go to a CPU host swap
pool over PCIe and come back when it resumes (src/mini_infra/core/types.py:110-114,
src/mini_infra/core/scheduler.py:312-313).  Its pool layout is per layer ``[num_blocks, bs, H, D]``
for K and V (src/mini_infra/worker/paged_kv_cache.py:23-52), so one block is ``2 * num_layers``
pieces spread over the pool.

Here a block travels as one **record**: ``[num_layers, 2 (K, V), bs, H, D]``, contiguous
(1.75 MiB for Qwen3-0.6B at block size 16).  ``mi_pack_blocks`` gathers blocks into records in
HBM and ``mi_unpack_blocks`` scatters records into (possibly other) blocks, so that:

* a swap is one HIP pack launch plus DMA copies of whole records into pinned host memory (no
  kernel reads or writes host memory), and a swap-in is the reverse;
* a file is a 64-byte header followed by the records.  Header, little-endian::

      0  8s  magic b"MIKVBLK1"        36  I  element bytes
      8  I   header bytes (64)        40  Q  number of records
     12  I   format version (1)       48  Q  record bytes
     16  I   num_layers               56  I  CRC-32 (zlib) of the record bytes
     20  I   block_size               60  I  reserved (0)
     24  I   num_kv_heads
     28  I   head_dim
     32  I   dtype code (1 bf16, 2 fp16, 3 fp32)

Every call runs on the current stream.  Host memory of a swap-out is valid after that stream has
passed it (``HostSwapPool.synchronize``); device blocks freed after a swap-out or a swap-in can be
reused by later work on the same stream at once.
"""

from __future__ import annotations

import math
import struct
import zlib
from collections import deque
from collections.abc import Sequence
from dataclasses import dataclass
from pathlib import Path

import torch

RECORD_MAGIC = b"MIKVBLK1"
FORMAT_VERSION = 1
_HEADER = struct.Struct("<8sIIIIIIIIQQII")
HEADER_BYTES = _HEADER.size  # 64
DTYPE_CODES = {torch.bfloat16: 1, torch.float16: 2, torch.float32: 3}
_CODE_DTYPES = {code: dtype for dtype, code in DTYPE_CODES.items()}


@dataclass(frozen=True)
class KVBlockHeader:
    """Geometry of a file of KV block records (and of the pool they come from)."""

    num_layers: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    num_records: int
    crc32: int = 0

    @property
    def element_bytes(self) -> int:
        return torch.empty((), dtype=self.dtype).element_size()

    @property
    def record_bytes(self) -> int:
        return 2 * self.num_layers * self.block_size * self.num_kv_heads * self.head_dim * self.element_bytes

    @property
    def record_shape(self) -> tuple[int, ...]:
        return (self.num_layers, 2, self.block_size, self.num_kv_heads, self.head_dim)

    def encode(self) -> bytes:
        if self.dtype not in DTYPE_CODES:
            raise ValueError(f"no record dtype code for {self.dtype}")
        return _HEADER.pack(RECORD_MAGIC, HEADER_BYTES, FORMAT_VERSION, self.num_layers, self.block_size,
                            self.num_kv_heads, self.head_dim, DTYPE_CODES[self.dtype], self.element_bytes,
                            self.num_records, self.record_bytes, self.crc32 & 0xFFFFFFFF, 0)

    @classmethod
    def decode(cls, raw: bytes) -> KVBlockHeader:
        if len(raw) < HEADER_BYTES:
            raise ValueError(f"KV block header needs {HEADER_BYTES} bytes, got {len(raw)}")
        (magic, header_bytes, version, layers, block_size, heads, head_dim, code, elt, n, record_bytes, crc,
         _reserved) = _HEADER.unpack(raw[:HEADER_BYTES])
        if magic != RECORD_MAGIC:
            raise ValueError(f"not a KV block record file (magic {magic!r})")
        if version != FORMAT_VERSION or header_bytes != HEADER_BYTES:
            raise ValueError(f"unsupported KV block record format version {version} / header {header_bytes} B")
        if code not in _CODE_DTYPES:
            raise ValueError(f"unknown record dtype code {code}")
        header = cls(layers, block_size, heads, head_dim, _CODE_DTYPES[code], n, crc)
        if min(layers, block_size, heads, head_dim) < 1 or elt != header.element_bytes \
                or record_bytes != header.record_bytes:
            raise ValueError("inconsistent KV block record header")
        return header


def pool_header(pool, num_records: int, crc32: int = 0) -> KVBlockHeader:
    """Header describing records of ``pool`` (a PagedKVCachePool)."""
    return KVBlockHeader(len(pool.kv_pools), pool.block_size, pool.num_kv_heads, pool.head_dim, pool.storage.dtype,
                         num_records, crc32)


def check_block_ids(pool, block_ids: Sequence[int], unique: bool) -> list[int]:
    ids = [int(b) for b in block_ids]
    for b in ids:
        if not 0 <= b < pool.num_blocks:
            raise ValueError(f"block id {b} outside the pool's [0, {pool.num_blocks})")
    if unique and len(set(ids)) != len(ids):
        raise ValueError("block ids written by one call must be unique")
    return ids


def _runs(slots: Sequence[int]) -> list[tuple[int, int, int]]:
    """(first slot, first index, length) of each run of consecutive slots."""
    runs: list[tuple[int, int, int]] = []
    for i, s in enumerate(slots):
        if runs and runs[-1][0] + runs[-1][2] == s:
            first, index, length = runs[-1]
            runs[-1] = (first, index, length + 1)
        else:
            runs.append((s, i, 1))
    return runs


class HostSwapPool:
    """CPU host swap pool: ``num_slots`` records of one pool geometry in pinned host memory.

    Slots are handed out FIFO like the device blocks of FreeKVCacheBlockQueue
    (src/mini_infra/core/block_manager.py:35-76); running out raises ``RuntimeError``.
    """

    def __init__(self, num_slots: int, pool):
        if num_slots < 1:
            raise ValueError("HostSwapPool needs at least one slot")
        self.header = pool_header(pool, 0)
        self.records = torch.empty((num_slots, *self.header.record_shape), dtype=pool.storage.dtype,
                                   pin_memory=True)
        self._free: deque[int] = deque(range(num_slots))
        self._done: torch.cuda.Event | None = None

    @property
    def num_slots(self) -> int:
        return self.records.shape[0]

    @property
    def num_free_slots(self) -> int:
        return len(self._free)

    def _check_pool(self, pool) -> None:
        if pool_header(pool, 0) != self.header:
            raise ValueError("pool geometry differs from the swap pool's")

    def allocate(self, n: int) -> list[int]:
        if n > len(self._free):
            raise RuntimeError(f"host swap pool out of slots: need {n}, have {len(self._free)}")
        return [self._free.popleft() for _ in range(n)]

    def free(self, slots: Sequence[int]) -> None:
        self._free.extend(int(s) for s in slots)

    def swap_out(self, pool, block_ids: Sequence[int]) -> list[int]:
        """Copies blocks ``block_ids`` (all layers) into newly allocated host slots; returns the slots.

        One pack launch into HBM, then one DMA copy per run of consecutive slots, all on the
        current stream.  The device blocks may be freed and reused by later work on that stream.
        """
        self._check_pool(pool)
        ids = check_block_ids(pool, block_ids, unique=False)
        slots = self.allocate(len(ids))
        if not ids:
            return slots
        staged = pool.pack_blocks(ids)
        for first, index, length in _runs(slots):
            self.records[first:first + length].copy_(staged[index:index + length], non_blocking=True)
        self._record(pool.device)
        return slots

    def swap_in(self, pool, slots: Sequence[int], block_ids: Sequence[int], free_slots: bool = True) -> None:
        """Copies host slots back into blocks ``block_ids`` (unique) of every layer, on the current
        stream; the slots are released unless ``free_slots`` is False."""
        self._check_pool(pool)
        slots = [int(s) for s in slots]
        ids = check_block_ids(pool, block_ids, unique=True)
        if len(slots) != len(ids):
            raise ValueError(f"{len(slots)} slots for {len(ids)} blocks")
        for s in slots:
            if not 0 <= s < self.num_slots:
                raise ValueError(f"slot {s} outside [0, {self.num_slots})")
        if ids:
            staged = torch.empty((len(ids), *self.header.record_shape), dtype=self.records.dtype, device=pool.device)
            for first, index, length in _runs(slots):
                staged[index:index + length].copy_(self.records[first:first + length], non_blocking=True)
            pool.unpack_blocks(staged, ids)
            self._record(pool.device)
        if free_slots:
            self.free(slots)

    def _record(self, device: torch.device) -> None:
        self._done = torch.cuda.Event()
        self._done.record(torch.cuda.current_stream(device))

    def synchronize(self) -> None:
        """Waits until every copy issued so far has finished (host slots readable / reusable by the CPU)."""
        if self._done is not None:
            self._done.synchronize()


def save_kv_blocks(path: str | Path, pool, block_ids: Sequence[int]) -> KVBlockHeader:
    """Writes blocks ``block_ids`` of every layer to ``path``: header + records (format above)."""
    ids = check_block_ids(pool, block_ids, unique=False)
    host = torch.empty((len(ids), *pool_header(pool, 0).record_shape), dtype=pool.storage.dtype, pin_memory=True)
    if ids:
        host.copy_(pool.pack_blocks(ids), non_blocking=True)
        torch.cuda.current_stream(pool.device).synchronize()
    payload = host.view(torch.uint8).numpy().reshape(-1) if host.numel() else memoryview(b"")
    header = pool_header(pool, len(ids), zlib.crc32(payload))
    with open(path, "wb") as f:
        f.write(header.encode())
        f.write(payload)
    return header


def load_kv_blocks(path: str | Path, pool, block_ids: Sequence[int]) -> KVBlockHeader:
    """Reads a record file into blocks ``block_ids`` (unique, one per record) of every layer.

    Raises ``ValueError`` on a bad header, a geometry that differs from the pool's, a short file
    or a CRC mismatch; the pool is written only after every check has passed.
    """
    ids = check_block_ids(pool, block_ids, unique=True)
    with open(path, "rb") as f:
        header = KVBlockHeader.decode(f.read(HEADER_BYTES))
        expect = pool_header(pool, header.num_records, header.crc32)
        if header != expect:
            raise ValueError(f"record file geometry {header} does not match the pool's {expect}")
        if header.num_records != len(ids):
            raise ValueError(f"file holds {header.num_records} records, {len(ids)} block ids given")
        host = torch.empty((len(ids), *header.record_shape), dtype=pool.storage.dtype, pin_memory=True)
        payload = host.view(torch.uint8).numpy().reshape(-1) if host.numel() else bytearray()
        got = f.readinto(memoryview(payload)) if len(ids) else 0
        if got != math.prod(host.shape) * host.element_size():
            raise ValueError(f"record file is short: {got} payload bytes")
        if f.read(1):
            raise ValueError("record file has trailing bytes")
    if zlib.crc32(payload) != header.crc32:
        raise ValueError("record file CRC-32 mismatch")
    if ids:
        pool.unpack_blocks(host.to(pool.device, non_blocking=True), ids)
        torch.cuda.current_stream(pool.device).synchronize()
    return header


__all__ = [
    "FORMAT_VERSION",
    "HEADER_BYTES",
    "HostSwapPool",
    "KVBlockHeader",
    "RECORD_MAGIC",
    "load_kv_blocks",
    "pool_header",
    "save_kv_blocks",
]
