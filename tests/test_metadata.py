"""Host metadata packing: known answers from the reference's suite and agreement with the
oracle's per-token loops on seeded random cases."""

import random

import numpy as np
import pytest

from mini_infra_qwen3_amd.core import KVCacheManager
from mini_infra_qwen3_amd.worker.metadata import (
    pack_decode_rows,
    pack_prefill_rows,
    padded_tables,
    prefill_scatter_indices,
)
from oracle import closed_form, torch_ref


def test_decode_rows_known_answer():
    """tests/unit/test_paged_kv_cache.py:96-106: A at position 5 in blocks [9, 4], B at 2 in [7]."""
    rows = pack_decode_rows([[9, 4], [7]], last_tokens=[11, 22], positions=[5, 2], block_size=4)
    assert rows[:, 0].tolist() == [11, 22] and rows[:, 1].tolist() == [5, 2]
    assert rows[:, 2].tolist() == [4 * 4 + 1, 7 * 4 + 2]
    assert rows[:, 3].tolist() == [6, 3]
    assert rows[:, 4:].tolist() == [[9, 4], [7, 0]]


def test_decode_rows_smoke_known_answer():
    """verification/smoke.py:320-336: position 6 of a 2-block table -> block[1] * 4 + 2, context 7."""
    rows = pack_decode_rows([[1, 2]], [7], [6], 4)
    assert rows[0, 2] == 2 * 4 + 2 and rows[0, 3] == 7


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_decode_rows_match_reference_loop(seed, block_size):
    rng = random.Random(seed)
    manager = KVCacheManager(block_size, num_blocks=512)
    positions = []
    for i in range(rng.randint(1, 9)):
        n = rng.randint(1, 60)
        assert manager.allocate_slots(i, n)
        positions.append(n - 1)
    tables = [manager.block_table(i) for i in range(len(positions))]
    tokens = [rng.randint(0, 1000) for _ in positions]
    ours = pack_decode_rows(tables, tokens, positions, block_size)
    ref = torch_ref.prepare_decode_rows(tables, tokens, positions, block_size).numpy()
    assert np.array_equal(ours, ref)


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_scatter_indices_match_reference_loop(seed, block_size):
    rng = random.Random(100 + seed)
    manager = KVCacheManager(block_size, num_blocks=1024)
    manager.allocate_slots(999, rng.randint(0, 40))  # make tables non-contiguous
    chunk_lens, starts = [], []
    for i in range(rng.randint(1, 6)):
        start = rng.randint(0, 50)
        n = rng.randint(1, 40)
        assert manager.allocate_slots(i, start + n)
        starts.append(start)
        chunk_lens.append(n)
    tables = [manager.block_table(i) for i in range(len(starts))]
    padded = max(chunk_lens) + rng.randint(0, 3)
    ours = prefill_scatter_indices(tables, chunk_lens, starts, padded, block_size)
    ref = np.array(torch_ref.store_prefill_indices(tables, chunk_lens, starts, padded, block_size), dtype=np.int64)
    assert np.array_equal(ours, ref.reshape(3, -1))
    # every slot is where the closed form puts logical position start + t
    k = 0
    for row, (table, n, start) in enumerate(zip(tables, chunk_lens, starts)):
        for t in range(n):
            assert ours[2, k] == closed_form.slot_of(table, start + t, block_size)
            k += 1
    assert len(set(ours[2].tolist())) == ours.shape[1]


def test_prefill_rows_layout():
    """Row layout of src/mini_infra/worker/paged_runner.py:57-72 on a two-row chunk step."""
    rows = pack_prefill_rows([[5, 6, 7], [8]], start_positions=[5, 2], block_tables=[[3, 4, 9], [6, 1]],
                             block_size=4, pad_token_id=0)
    width = 3
    assert rows[:, :width].tolist() == [[5, 6, 7], [0, 0, 8]]
    assert rows[:, width:2 * width].tolist() == [[5, 6, 7], [0, 0, 2]]
    assert rows[:, 2 * width:2 * width + 2].tolist() == [[5, 3], [2, 1]]
    assert rows[:, 2 * width + 2:].tolist() == [[3, 4], [6, 0]]  # ceil(5/4)=2 and ceil(2/4)=1 blocks


def test_tables_cover_positions():
    with pytest.raises(ValueError):
        pack_decode_rows([[1]], [0], [4], 4)
    with pytest.raises(ValueError):
        prefill_scatter_indices([[1]], [2], [3], 2, 4)
    assert padded_tables([[1, 2], []]).tolist() == [[1, 2], [0, 0]]
