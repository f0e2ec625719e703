"""Control-plane block allocator: the known-answer sequences of the reference's own suite
(tests/unit/test_block_manager.py:16-129), re-expressed for this package."""

import pytest

from mini_infra_qwen3_amd.core import (
    NULL_BLOCK_ID,
    FreeKVCacheBlockQueue,
    KVCacheManager,
    PagedCacheConfig,
    Request,
    num_blocks_for_tokens,
    required_pool_blocks,
)


def test_num_blocks_for_tokens_is_ceil():
    assert [num_blocks_for_tokens(n, 4) for n in (1, 4, 5, 8, 9)] == [1, 1, 2, 2, 3]
    assert num_blocks_for_tokens(0, 16) == 0


def test_queue_skips_null_block_and_reuses_in_fifo_order():
    queue = FreeKVCacheBlockQueue(num_blocks=5)
    assert (queue.num_free_blocks, queue.num_used_blocks) == (4, 0)
    first = queue.allocate(3)
    assert first == [1, 2, 3] and NULL_BLOCK_ID not in first
    assert (queue.num_free_blocks, queue.num_used_blocks) == (1, 3)
    queue.free([2, 1])
    assert queue.allocate(3) == [4, 2, 1]  # never-used 4 first, then 2 and 1 in release order
    with pytest.raises(RuntimeError):
        queue.allocate(1)


def test_queue_needs_an_allocatable_block():
    with pytest.raises(ValueError, match="num_blocks"):
        FreeKVCacheBlockQueue(num_blocks=1)


def test_allocate_slots_grows_only_at_block_boundaries():
    manager = KVCacheManager(block_size=4, num_blocks=8)
    assert manager.allocate_slots(7, 5)
    assert manager.block_table(7) == [1, 2]
    for _ in range(3):
        assert manager.allocate_slots(7, 1)
    assert manager.block_table(7) == [1, 2]
    assert manager.allocate_slots(7, 1)  # token 9 opens block 3
    assert manager.block_table(7) == [1, 2, 3]
    assert manager.num_used_blocks == 3


def test_failed_allocation_leaves_no_state():
    manager = KVCacheManager(block_size=2, num_blocks=4)
    assert manager.allocate_slots(0, 4)
    assert not manager.allocate_slots(1, 4)
    assert manager.num_used_blocks == 2
    with pytest.raises(KeyError):
        manager.block_table(1)
    assert not manager.allocate_slots(0, 3)
    assert manager.block_table(0) == [1, 2]
    assert manager.allocate_slots(1, 2)


def test_free_returns_blocks():
    manager = KVCacheManager(block_size=2, num_blocks=4)
    manager.allocate_slots(0, 4)
    manager.allocate_slots(1, 2)
    manager.free(0)
    assert manager.num_used_blocks == 1
    with pytest.raises(KeyError):
        manager.block_table(0)
    assert manager.allocate_slots(2, 4)
    assert sorted(manager.block_table(1) + manager.block_table(2)) == [1, 2, 3]


def test_num_admissible_is_an_fcfs_prefix():
    manager = KVCacheManager(block_size=4, num_blocks=6)
    assert manager.num_admissible([8, 4, 4], 0) == 3
    assert manager.num_admissible([8, 12, 1], 0) == 2
    assert manager.num_admissible([24, 4], 0) == 0
    assert manager.num_admissible([], 0) == 0
    assert manager.num_admissible([8, 4, 4], 2) == 2


def test_required_pool_blocks_sums_longest_concurrent_requests():
    requests = [Request(0, (1,) * 5, 4), Request(1, (1,) * 3, 2), Request(2, (1,) * 9, 1)]
    assert required_pool_blocks(requests, 2, 4) == 1 + 3 + 2
    assert required_pool_blocks(requests, 8, 4) == 1 + 3 + 2 + 1


def test_paged_cache_config_validates():
    assert PagedCacheConfig().block_size == 16 and PagedCacheConfig().num_blocks is None
    with pytest.raises(ValueError, match="block_size"):
        PagedCacheConfig(block_size=0)
    with pytest.raises(ValueError, match="num_blocks"):
        PagedCacheConfig(num_blocks=1)


def test_counters_track_cold_reuse_release_and_peak():
    manager = KVCacheManager(block_size=4, num_blocks=5)
    assert (manager.block_cold_allocation_count, manager.block_reuse_count,
            manager.block_release_count, manager.peak_used_blocks) == (0, 0, 0, 0)
    assert manager.allocate_slots(0, 8)
    assert (manager.block_cold_allocation_count, manager.block_reuse_count, manager.peak_used_blocks) == (2, 0, 2)
    manager.free(0)
    assert manager.block_release_count == 2 and manager.num_used_blocks == 0
    assert manager.allocate_slots(1, 12)  # cold 3, 4 then warm 1
    assert (manager.block_cold_allocation_count, manager.block_reuse_count, manager.peak_used_blocks) == (4, 1, 3)
    assert manager.block_table(1) == [3, 4, 1]


def test_smoke_reuse_sequence():
    """Free-queue trajectory of the reference's paged smoke check (verification/smoke.py:299-352)."""
    manager = KVCacheManager(block_size=4, num_blocks=4)
    assert manager.allocate_slots(0, 6)
    old = list(manager.block_table(0))
    assert old == [1, 2]
    assert manager.allocate_slots(0, 1) and len(manager.block_table(0)) == 2
    manager.free(0)
    assert manager.allocate_slots(99, 2) and manager.block_table(99) == [3]
    assert manager.allocate_slots(1, 2) and manager.block_table(1)[0] == min(old)
    assert manager.block_reuse_count == 1


@pytest.mark.parametrize("seed,block_size,num_blocks", [(0, 16, 300), (1, 4, 64), (2, 1, 40), (3, 16, 5000)])
def test_matches_the_reference_allocator_under_random_churn(seed, block_size, num_blocks):
    """Thousands of seeded admissions, growth steps and frees against the oracle's restatement of the
    reference allocator (deque + set + lists, oracle/control_ref.py): every table, every counter and
    every success / failure identical; the delta log rebuilds the table matrix."""
    import random

    import numpy as np

    from oracle.control_ref import ReferenceBlockAllocator

    rng = random.Random(seed)
    mine, ref = KVCacheManager(block_size, num_blocks), ReferenceBlockAllocator(block_size, num_blocks)
    mirror = np.zeros((0, 0), dtype=np.int64)
    live: list[int] = []
    next_idx = 0
    for step in range(4000):
        op = rng.random()
        if op < 0.35 or not live:
            n = rng.randint(0, 6 * block_size)
            assert mine.allocate_slots(next_idx, n) == ref.allocate_slots(next_idx, n)
            if next_idx in ref.tables:
                live.append(next_idx)
            next_idx += 1
        elif op < 0.8:
            idx = rng.choice(live)
            n = rng.choice([1, 1, 1, rng.randint(1, 3 * block_size)])
            assert mine.allocate_slots(idx, n) == ref.allocate_slots(idx, n)
        else:
            idx = live.pop(rng.randrange(len(live)))
            mine.free(idx)
            ref.free(idx)
        lens = [rng.randint(1, 8 * block_size) for _ in range(rng.randint(0, 6))]
        reserved = rng.randint(-2, 10)
        assert mine.num_admissible(lens, reserved) == ref.num_admissible(lens, reserved)
        assert (mine.num_used_blocks, mine.block_cold_allocation_count, mine.block_reuse_count,
                mine.block_release_count, mine.peak_used_blocks) == (ref.used, ref.cold, ref.reuse, ref.release,
                                                                     ref.peak)
        rows, cols, ids = mine.take_deltas()
        shape = mine.table_matrix.shape
        if mirror.shape != shape:
            grown = np.zeros(shape, dtype=np.int64)
            grown[:mirror.shape[0], :mirror.shape[1]] = mirror
            mirror = grown
        mirror[rows, cols] = ids
        if step % 50 == 0 or step == 3999:
            for idx in live:
                table = ref.tables[idx]
                assert mine.block_table(idx) == table
                assert mirror[mine.row_of(idx), :len(table)].tolist() == table


def test_device_block_tables_follow_the_allocator_by_deltas():
    """The persistent table copy (here on the CPU device) equals every live request's table after
    each sync, uploading only the entries written since the previous one."""
    import random

    from mini_infra_qwen3_amd.worker.block_tables import DeviceBlockTables

    rng = random.Random(5)
    manager = KVCacheManager(16, 400)
    assert manager.allocate_slots(100, 40)  # written before the copy exists: uploaded whole
    tables = DeviceBlockTables(manager, max_rows=32, max_blocks=64, device="cpu")
    live = [100]
    uploaded = 0
    for step in range(600):
        if rng.random() < 0.2 and len(live) < 30:
            idx = 1000 + step
            if manager.allocate_slots(idx, rng.randint(1, 300)):
                live.append(idx)
        elif rng.random() < 0.1 and len(live) > 1:
            manager.free(live.pop(rng.randrange(len(live))))
        for idx in live:  # a decode step: one token each
            manager.allocate_slots(idx, 1)
        uploaded += tables.sync()
        for idx in live:
            table = manager.block_table(idx)
            assert tables.tensor[manager.row_of(idx), :len(table)].tolist() == table
    assert uploaded == tables.uploaded_entries < 600 * 10  # deltas, not whole tables every step
    small = KVCacheManager(16, 100)
    narrow = DeviceBlockTables(small, max_rows=4, max_blocks=4, device="cpu")
    assert small.allocate_slots(0, 16 * 5)
    with pytest.raises(ValueError, match="outside the device copy"):
        narrow.sync()
