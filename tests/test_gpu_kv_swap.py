"""KV block records on the GPU: mi_pack_blocks / mi_unpack_blocks bit-exact against the oracle's
record restatement, swaps through pinned host memory, the record file, and a decode that resumes
after its blocks went to the host and came back in other physical blocks (the "swap" preemption
mode the reference plans: src/mini_infra/core/types.py:110-114, core/scheduler.py:312-313)."""

import numpy as np
import pytest
import torch

from mini_infra_qwen3_amd import data_plane
from mini_infra_qwen3_amd.core import KVCacheManager
from mini_infra_qwen3_amd.model import Qwen3Config, Qwen3ForCausalLM, init_random_
from mini_infra_qwen3_amd.worker import (HostSwapPool, KVBlockHeader, PagedKVCachePool, PagedRunner,
                                         load_kv_blocks, save_kv_blocks)
from oracle import closed_form

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def bits(t):
    t = t.contiguous().cpu()
    return t.view(torch.int16).numpy() if t.element_size() == 2 else t.view(torch.int32).numpy()


def random_pool(layers, num_blocks, bs=16, heads=8, dim=128, dtype=torch.bfloat16, seed=0):
    pool = PagedKVCachePool(layers, num_blocks, bs, heads, dim, dtype, DEV)
    g = torch.Generator().manual_seed(seed)
    pool.storage.copy_(torch.randn(pool.storage.shape, generator=g).to(dtype))
    return pool


def pool_bits(pool):
    return [bits(k) for k, _ in pool.kv_pools], [bits(v) for _, v in pool.kv_pools]


@pytest.mark.parametrize("layers,bs,heads,dim,dtype", [
    (28, 16, 8, 128, torch.bfloat16),   # Qwen3-0.6B
    (33, 16, 8, 128, torch.bfloat16),   # two launches (32 layers per launch)
    (2, 32, 8, 128, torch.bfloat16),
    (3, 16, 4, 64, torch.float32),
    (2, 1, 1, 2, torch.bfloat16),       # 4-byte pieces
    (2, 1, 1, 3, torch.bfloat16),       # 2-byte pieces
], ids=["qwen3", "33layers", "block32", "fp32", "piece4", "piece2"])
def test_pack_matches_oracle(native_lib, layers, bs, heads, dim, dtype):
    nb = 40
    pool = random_pool(layers, nb, bs, heads, dim, dtype, seed=layers)
    ids = [7, 0, 39, 7, 12, 3, 38, 21]
    records = pool.pack_blocks(ids)
    assert tuple(records.shape) == (len(ids), layers, 2, bs, heads, dim)
    keys, values = pool_bits(pool)
    assert np.array_equal(bits(records), closed_form.pack_records(keys, values, ids))


def test_pack_of_out_of_range_ids_reads_the_null_block(native_lib):
    pool = random_pool(2, 10)
    ids = torch.tensor([3, -1, 10, 1 << 40, 9], dtype=torch.long, device=DEV)
    records = data_plane.pack_blocks([k for k, _ in pool.kv_pools], [v for _, v in pool.kv_pools], ids)
    keys, values = pool_bits(pool)
    assert np.array_equal(bits(records), closed_form.pack_records(keys, values, ids.tolist()))
    zero = data_plane.pack_blocks([k for k, _ in pool.kv_pools], [v for _, v in pool.kv_pools],
                                  torch.zeros(1, dtype=torch.long, device=DEV))
    for i in (1, 2, 3):
        assert torch.equal(records[i], zero[0])


def test_unpack_matches_oracle_and_leaves_other_blocks(native_lib):
    pool = random_pool(28, 64, seed=3)
    g = torch.Generator().manual_seed(4)
    records = torch.randn((6, 28, 2, 16, 8, 128), generator=g).to(torch.bfloat16)
    ids = [5, 63, 1, 17, 40, 2]
    keys, values = pool_bits(pool)
    pool.unpack_blocks(records.to(DEV), ids)
    want_k, want_v = closed_form.unpack_records(keys, values, bits(records), ids)
    got_k, got_v = pool_bits(pool)
    for layer in range(28):
        assert np.array_equal(got_k[layer], want_k[layer]) and np.array_equal(got_v[layer], want_v[layer])


def test_unpack_skips_out_of_range_ids(native_lib):
    pool = random_pool(2, 8, seed=5)
    before = pool.storage.clone()
    records = torch.ones((3, 2, 2, 16, 8, 128), dtype=torch.bfloat16, device=DEV)
    ids = torch.tensor([-3, 8, 2], dtype=torch.long, device=DEV)
    data_plane.unpack_blocks(records, [k for k, _ in pool.kv_pools], [v for _, v in pool.kv_pools], ids)
    after = pool.storage.clone()
    assert torch.equal(after[:, :, 2], torch.ones_like(after[:, :, 2]))
    keep = [b for b in range(8) if b != 2]
    assert np.array_equal(bits(after[:, :, keep]), bits(before[:, :, keep]))


def test_pack_unpack_round_trip_into_other_blocks(native_lib):
    pool = random_pool(28, 300, seed=6)
    g = torch.Generator().manual_seed(7)
    perm = torch.randperm(299, generator=g)[:128] + 1
    src, dst = perm[:64].tolist(), perm[64:].tolist()
    before = pool.storage.clone()
    pool.unpack_blocks(pool.pack_blocks(src), dst)
    after = pool.storage
    assert np.array_equal(bits(after[:, :, dst]), bits(before[:, :, src]))
    keep = sorted(set(range(300)) - set(dst))
    assert np.array_equal(bits(after[:, :, keep]), bits(before[:, :, keep]))


def test_host_checks_of_block_ids(native_lib):
    pool = random_pool(2, 8)
    with pytest.raises(ValueError, match="unique"):
        pool.unpack_blocks(pool.pack_blocks([1, 2]), [3, 3])
    with pytest.raises(ValueError):
        pool.pack_blocks([8])
    with pytest.raises(ValueError):
        pool.unpack_blocks(pool.pack_blocks([1]), [1, 2])
    assert pool.pack_blocks([]).shape == (0, 2, 2, 16, 8, 128)


def test_host_swap_pool_round_trip_with_slot_reuse(native_lib):
    pool = random_pool(28, 200, seed=8)
    swap = HostSwapPool(40, pool)
    original = pool.storage.clone()
    a = swap.swap_out(pool, [10, 11, 12, 50, 3])
    b = swap.swap_out(pool, list(range(100, 130)))
    assert swap.num_free_slots == 5 and a == [0, 1, 2, 3, 4]
    with pytest.raises(RuntimeError, match="out of slots"):
        swap.swap_out(pool, list(range(6)))
    swap.synchronize()
    pool.storage.normal_()  # the device blocks are reused for something else
    swap.swap_in(pool, a, [150, 151, 152, 153, 154])
    assert swap.num_free_slots == 10
    c = swap.swap_out(pool, [1, 2, 3, 4, 5, 6, 7])  # reuses freed slots (FIFO: 35..39, then 0, 1)
    assert c == [35, 36, 37, 38, 39, 0, 1]
    swap.swap_in(pool, b[::-1], list(range(160, 190)))
    got = pool.storage
    assert np.array_equal(bits(got[:, :, 150:155]), bits(original[:, :, [10, 11, 12, 50, 3]]))
    assert np.array_equal(bits(got[:, :, 160:190]), bits(original[:, :, list(range(129, 99, -1))]))
    with pytest.raises(ValueError):
        swap.swap_in(pool, c[:2], [1])
    other = random_pool(27, 10)
    with pytest.raises(ValueError, match="geometry"):
        swap.swap_out(other, [1])


def test_record_file_round_trip_and_corruption(native_lib, tmp_path):
    pool = random_pool(28, 64, seed=9)
    ids = [4, 9, 33, 4]
    path = tmp_path / "blocks.kv"
    header = save_kv_blocks(path, pool, ids)
    raw = path.read_bytes()
    assert len(raw) == 64 + 4 * pool.bytes_per_block
    assert KVBlockHeader.decode(raw[:64]) == header and header.num_records == 4
    keys, values = pool_bits(pool)
    assert np.array_equal(np.frombuffer(raw[64:], dtype=np.int16).reshape(4, 28, 2, 16, 8, 128),
                          closed_form.pack_records(keys, values, ids))
    dst = random_pool(28, 20, seed=10)
    load_kv_blocks(path, dst, [19, 1, 7, 2])
    assert np.array_equal(bits(dst.storage[:, :, [19, 1, 7, 2]]), bits(pool.storage[:, :, ids]))
    before = dst.storage.clone()
    bad = bytearray(raw)
    bad[64 + 123456] ^= 0x40
    path.write_bytes(bytes(bad))
    with pytest.raises(ValueError, match="CRC"):
        load_kv_blocks(path, dst, [3, 4, 5, 6])
    path.write_bytes(raw[:-1])
    with pytest.raises(ValueError, match="short"):
        load_kv_blocks(path, dst, [3, 4, 5, 6])
    path.write_bytes(raw)
    with pytest.raises(ValueError, match="geometry"):
        load_kv_blocks(path, random_pool(28, 20, bs=32), [3, 4, 5, 6])
    with pytest.raises(ValueError, match="records"):
        load_kv_blocks(path, dst, [3, 4, 5])
    assert np.array_equal(bits(dst.storage), bits(before))
    empty = tmp_path / "empty.kv"
    assert save_kv_blocks(empty, pool, []).num_records == 0
    assert load_kv_blocks(empty, dst, []).num_records == 0


def test_decode_resumes_after_swap_to_other_blocks(native_lib):
    """Three requests decode 4 steps, go to the host swap pool, their blocks are freed and written
    over by another request, they come back into other blocks and decode 4 more steps: the tokens
    equal those of an uninterrupted run on a second pool."""
    cfg = Qwen3Config(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128)
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, seed=0, std=0.05, untied_head_seed=1234)
    model = model.to(torch.bfloat16).to(DEV).eval()
    runner = PagedRunner(model)
    gen = torch.Generator().manual_seed(3)
    prompts = [torch.randint(1, 999, (n,), generator=gen).tolist() for n in (37, 16, 5)]

    def start(manager, pool):
        for i, p in enumerate(prompts):
            manager.allocate_slots(i, len(p))
        tables = [manager.block_table(i) for i in range(3)]
        out = runner.run_prefill_step(prompts)
        runner.store_prefill(pool, out.prefill_cache, tables, [len(p) for p in prompts], [0] * 3)
        return [[t] for t in out.next_tokens], [len(p) for p in prompts]

    def decode(manager, pool, tokens, lengths, steps):
        for _ in range(steps):
            for i in range(3):
                assert manager.allocate_slots(i, 1)
            tables = [manager.block_table(i) for i in range(3)]
            ids, pos, meta = runner.prepare_decode_inputs(tables, [t[-1] for t in tokens], lengths, 16)
            out = runner.run_decode_step(ids, pos, meta, pool)
            for i in range(3):
                lengths[i] += 1
                tokens[i].append(out.next_tokens[i])

    with torch.inference_mode():
        ref_manager, ref_pool = KVCacheManager(16, num_blocks=64), PagedKVCachePool(2, 64, 16, 8, 128,
                                                                                    torch.bfloat16, DEV)
        ref_tokens, ref_lengths = start(ref_manager, ref_pool)
        decode(ref_manager, ref_pool, ref_tokens, ref_lengths, 8)

        manager, pool = KVCacheManager(16, num_blocks=64), PagedKVCachePool(2, 64, 16, 8, 128, torch.bfloat16, DEV)
        swap = HostSwapPool(16, pool)
        tokens, lengths = start(manager, pool)
        decode(manager, pool, tokens, lengths, 4)
        slots = {i: swap.swap_out(pool, manager.block_table(i)) for i in range(3)}
        counts = {i: len(manager.block_table(i)) for i in range(3)}
        for i in range(3):
            manager.free(i)
        assert manager.allocate_slots(9, 16 * 40)  # another request takes and overwrites the freed blocks
        pool.storage.normal_()
        manager.free(9)
        for i in (2, 0, 1):
            assert manager.allocate_slots(i, lengths[i]) and len(manager.block_table(i)) == counts[i]
            swap.swap_in(pool, slots[i], manager.block_table(i))
        assert swap.num_free_slots == 16
        decode(manager, pool, tokens, lengths, 4)
    assert tokens == ref_tokens
