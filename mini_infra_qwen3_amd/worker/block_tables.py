"""Persistent device copy of the block tables, updated by deltas.

The reference packs every decoding request's whole block table into a fresh ``[B, 4 + max_blocks]``
int64 tensor and uploads it every step (src/mini_infra/worker/paged_runner.py:138-166).  Here the
tables live on the GPU for the whole run as one ``[rows, width]`` matrix, a copy of
``KVCacheManager.table_matrix``.  Before a step, ``sync()`` uploads only the entries the manager
wrote since the last step -- one id per request whenever it crosses a block boundary -- and the
step itself uploads ``[B, 5]`` per-row scalars (token, position, slot, context length, table row).
The decode forward gathers its rows on the device (``PagedAttentionMetadata.table_rows``).
"""

from __future__ import annotations

import numpy as np
import torch

from mini_infra_qwen3_amd.core.block_manager import KVCacheManager


class DeviceBlockTables:
    """``tensor``: ``[max_rows, max_blocks]`` int64 on ``device``, row r = the manager's row r.

    Entries past a request's blocks are the null block or ids of an earlier request of the row:
    the kernels read only the blocks a context covers.
    """

    def __init__(self, manager: KVCacheManager, max_rows: int, max_blocks: int, device: torch.device):
        self.manager = manager
        self.device = torch.device(device)
        self.tensor = torch.zeros((max(int(max_rows), 1), max(int(max_blocks), 1)), dtype=torch.long,
                                  device=self.device)
        manager.take_deltas()  # the full upload below covers everything written so far
        current = manager.table_matrix
        rows, width = min(current.shape[0], self.tensor.shape[0]), min(current.shape[1], self.tensor.shape[1])
        if (current[rows:] != 0).any() or (current[:, width:] != 0).any():
            raise ValueError(f"the manager's tables {current.shape} exceed the device copy {tuple(self.tensor.shape)}")
        self.tensor[:rows, :width] = torch.from_numpy(np.ascontiguousarray(current[:rows, :width])).to(self.device)
        self.uploaded_entries = 0

    def sync(self) -> int:
        """Uploads the entries written since the last call (one copy of ``[2, n]`` int64 and one
        scatter on the current stream); returns n."""
        rows, cols, ids = self.manager.take_deltas()
        n = int(rows.shape[0])
        if n == 0:
            return 0
        max_rows, width = self.tensor.shape
        if int(rows.max()) >= max_rows or int(cols.max()) >= width:
            raise ValueError(f"table entry ({int(rows.max())}, {int(cols.max())}) outside the device copy "
                             f"{tuple(self.tensor.shape)}")
        packed = torch.from_numpy(np.stack((rows * width + cols, ids))).to(self.device)
        self.tensor.view(-1).index_copy_(0, packed[0], packed[1])
        self.uploaded_entries += n
        return n


__all__ = ["DeviceBlockTables"]
