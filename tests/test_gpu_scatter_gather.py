"""Kernels 1 and 2 on the GPU: reshape-and-cache scatter and block-table gather must be
bit-exact against the oracle (the reference's index_copy_ / advanced-index chain on CPU)."""

import numpy as np
import pytest
import torch

from mini_infra_qwen3_amd import data_plane, workloads
from mini_infra_qwen3_amd.worker import KVCache, PagedKVCachePool
from oracle import closed_form, torch_ref

pytestmark = pytest.mark.gpu


def as_bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int16) if t.element_size() == 2 else t.contiguous().view(torch.int32)


def assert_bit_equal(a: torch.Tensor, b: torch.Tensor):
    assert a.shape == b.shape
    assert torch.equal(as_bits(a.cpu()), as_bits(b.cpu()))


# ------------------------------------------------------------------------------- scatter
def test_decode_append_matches_oracle_on_decode_step_workload(native_lib, device):
    """Batch 8, contexts U[64, 512], 4096-block pool: append of the new K/V row per sequence."""
    w = workloads.decode_step(seed=11)
    pools = w.pools.to(device)
    slots = w.slot_mapping
    new_k = w.new_key[0].unsqueeze(2)       # [B, Hkv, 1, D] contiguous like the reference key
    new_v = w.new_value[0].unsqueeze(2)
    data_plane.reshape_and_cache([new_k.to(device)], [new_v.to(device)], slots.to(device),
                                 [pools[0, 0]], [pools[0, 1]])
    ref_k, ref_v = w.pools[0, 0].clone(), w.pools[0, 1].clone()
    rows = new_k.view(-1, workloads.NUM_KV_HEADS, workloads.HEAD_DIM)
    ref_k.view(-1, 8, 128).index_copy_(0, slots, rows)
    ref_v.view(-1, 8, 128).index_copy_(0, slots, new_v.view(-1, 8, 128))
    assert_bit_equal(pools[0, 0], ref_k)
    assert_bit_equal(pools[0, 1], ref_v)


def test_prefill_scatter_matches_oracle_with_churned_tables(native_lib, device):
    """Prefill form over 3 layers, 6 prompts U[128, 600], churned tables, V as a transpose view."""
    w = workloads.prefill_scatter(seed=3, device=device, num_prompts=6, lo=128, hi=600, num_layers=3)
    pool = PagedKVCachePool(3, w.num_blocks, 16, 8, 128, torch.bfloat16, device)
    # pre-fill the pool so "untouched rows stay untouched" is a real check
    pool.storage.copy_(torch.randn(pool.storage.shape, device=device).to(torch.bfloat16))
    before = [(k.cpu(), v.cpu()) for k, v in pool.kv_pools]
    layers = []
    for layer in range(3):
        key = w.sources[layer, 0]
        # value as the reference produces it: v_proj(...).view(B, L, H, D).transpose(1, 2)
        value = w.sources[layer, 1].transpose(1, 2).contiguous().transpose(1, 2)
        layers.append((key, value))
    index = torch.from_numpy(w.index).to(device)
    pool.write_prefill(KVCache(layers), index[0], index[1], index[2])
    ref_pools = [(k.clone(), v.clone()) for k, v in before]
    cpu_layers = [(k.cpu(), v.cpu()) for k, v in layers]
    idx = torch.from_numpy(w.index)
    torch_ref.write_prefill(ref_pools, cpu_layers, idx[0], idx[1], idx[2])
    for (gk, gv), (rk, rv) in zip(pool.kv_pools, ref_pools):
        assert_bit_equal(gk, rk)
        assert_bit_equal(gv, rv)


def test_scatter_small_fp32_shape_and_narrow_pieces(native_lib, device):
    """Reference tiny-model shape (2 KV heads x head_dim 4, fp32: 16-byte heads) and an odd
    head_dim (6 x bf16: 12-byte heads, element-wise pieces) both match the closed form."""
    for heads, dim, dtype in ((2, 4, torch.float32), (3, 6, torch.bfloat16)):
        gen = torch.Generator().manual_seed(heads)
        src_k = torch.randn(3, heads, 7, dim, generator=gen).to(dtype)
        src_v = torch.randn(3, 7, heads, dim, generator=gen).to(dtype).transpose(1, 2)
        pool_k = torch.randn(6, 4, heads, dim, generator=gen).to(dtype)
        pool_v = torch.randn(6, 4, heads, dim, generator=gen).to(dtype)
        rows = torch.tensor([0, 0, 1, 2, 2])
        pos = torch.tensor([5, 6, 6, 2, 6])
        slots = torch.tensor([4, 5, 23, 9, 0])
        gk, gv = pool_k.to(device), pool_v.to(device)
        data_plane.reshape_and_cache([src_k.to(device)], [src_v.to(device)], slots.to(device), [gk], [gv],
                                     token_rows=rows.to(device), token_positions=pos.to(device))
        bits = (lambda t: t.contiguous().view(torch.int32 if dtype == torch.float32 else torch.int16).numpy())
        assert np.array_equal(bits(gk.cpu()), closed_form.scatter_rows(bits(pool_k), bits(src_k), rows, pos, slots))
        assert np.array_equal(bits(gv.cpu()), closed_form.scatter_rows(bits(pool_v), bits(src_v), rows, pos, slots))


def test_scatter_empty_and_out_of_range_slots(native_lib, device):
    pool_k = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16, device=device)
    pool_v = torch.zeros_like(pool_k)
    src = torch.ones(2, 8, 1, 128, dtype=torch.bfloat16, device=device)
    empty = torch.empty(0, dtype=torch.long, device=device)
    data_plane.reshape_and_cache([src], [src], empty, [pool_k], [pool_v])
    assert not pool_k.any()
    # slot 64 is one past the pool: skipped, never written out of bounds; slot 3 is written
    slots = torch.tensor([64, 3], device=device)
    data_plane.reshape_and_cache([src], [src * 2], slots, [pool_k], [pool_v])
    torch.cuda.synchronize()
    flat = pool_k.view(-1, 8, 128)
    assert flat[3].eq(1).all() and flat.sum().item() == 8 * 128
    assert pool_v.view(-1, 8, 128)[3].eq(2).all()


def test_scatter_rejects_cpu_tensors(native_lib):
    pool = torch.zeros(2, 16, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        data_plane.reshape_and_cache([pool[:1]], [pool[:1]], torch.zeros(1, dtype=torch.long), [pool], [pool])


@pytest.mark.parametrize("tables", ["fragmented", "near_sequential"])
def test_prefill_scatter_full_size_every_layer(native_lib, device, tables):
    """32 prompts U[128, 2048] x 28 layers (about 9.3 GB moved), on both table kinds: every
    written pool row of every layer equals its source row, read on the device with torch's own
    advanced indexing (not through the product's gather), and blocks in no table stay zero."""
    w = workloads.prefill_scatter(seed=0, device=device, tables=tables)
    if tables == "fragmented":
        assert workloads.consecutive_fraction(w.tables) < 0.01
    pool = PagedKVCachePool(28, w.num_blocks, 16, 8, 128, torch.bfloat16, device)
    layers = [(w.sources[l, 0], w.sources[l, 1]) for l in range(28)]
    index = torch.from_numpy(w.index).to(device)
    pool.write_prefill(KVCache(layers), index[0], index[1], index[2])
    rows, positions, slots = index[0], index[1], index[2]
    for layer in range(28):
        for kv in range(2):
            written = pool.kv_pools[layer][kv].view(-1, 8, 128)[slots]          # [N, Hkv, D]
            expected = w.sources[layer, kv][rows, :, positions, :]              # [N, Hkv, D]
            assert torch.equal(as_bits(written), as_bits(expected)), (layer, kv)
    # untouched blocks (never in any table) stay zero in every layer
    used = torch.zeros(w.num_blocks, dtype=torch.bool)
    for t in w.tables:
        used[torch.tensor(t)] = True
    free = (~used).nonzero().flatten().to(device)
    assert not pool.storage[:, :, free].any()
    # slots of a prompt's last block past its length stay zero too
    tails = [t[-1] * 16 + s for t, n in zip(w.tables, w.lengths) for s in range(n % 16 or 16, 16)]
    if tails:
        tail = torch.tensor(tails, device=device)
        assert not pool.storage.view(28, 2, -1, 8, 128)[:, :, tail].any()


# -------------------------------------------------------------------------------- gather
@pytest.mark.parametrize("tables", ["fragmented", "near_sequential"])
def test_history_gather_full_size_every_chunk(native_lib, device, tables):
    """The history gather of 4 prompts x 16384 tokens in 2048-token chunks, 28 layers, on both
    table kinds: chunk c gathers the first 128 c blocks of every prompt's table, and each gathered
    layer equals torch's own advanced indexing of the pool on the device, bit for bit."""
    w = workloads.chunked_prefill(seed=0, tables=tables)
    pool = PagedKVCachePool(28, w.num_blocks, 16, 8, 128, torch.bfloat16, device)
    pool.storage.view(torch.int16).random_(generator=torch.Generator(device=device).manual_seed(2))
    for c in range(1, w.num_chunks):
        nb = c * w.chunk_len // 16
        ids = torch.tensor([t[:nb] for t in w.tables], dtype=torch.long, device=device)
        got = pool.gather_blocks(ids)
        for layer in range(28):
            for kv in range(2):
                want = pool.kv_pools[layer][kv][ids].view(w.num_prompts, nb * 16, 8, 128).transpose(1, 2)
                assert torch.equal(as_bits(got[layer][kv]), as_bits(want)), (c, layer, kv)
        del got


def test_gather_matches_oracle_including_null_and_stale_blocks(native_lib, device):
    gen = torch.Generator().manual_seed(5)
    pool = PagedKVCachePool(4, 40, 16, 8, 128, torch.bfloat16, device)
    cpu = torch.randn(pool.storage.shape, generator=gen).to(torch.bfloat16)
    pool.storage.copy_(cpu)
    ids = torch.tensor([[3, 17, 0, 0], [39, 3, 3, 1], [0, 0, 0, 0]])
    got = pool.gather_blocks(ids.to(device))
    ref = torch_ref.gather_blocks([(cpu[l, 0], cpu[l, 1]) for l in range(4)], ids)
    for (gk, gv), (rk, rv) in zip(got, ref):
        assert gk.shape == rk.shape == (3, 8, 64, 128)
        assert gk.stride() == rk.stride()  # same transposed view of a [B, nb*16, H, D] buffer
        assert_bit_equal(gk, rk)
        assert_bit_equal(gv, rv)


def test_gather_tiny_fp32_arange_known_answer(native_lib, device):
    """tests/unit/test_paged_kv_cache.py:265-280 on the GPU (2 KV heads, head_dim 4, block 4, fp32)."""
    pool = PagedKVCachePool(2, 6, 4, 2, 4, torch.float32, device)
    for k, v in pool.kv_pools:
        k.copy_(torch.arange(k.numel(), dtype=torch.float32, device=device).view_as(k))
        v.copy_(k + 0.5)
    (key, value), _ = pool.gather_blocks(torch.tensor([[2, 4], [5, 0]], device=device))
    kp, vp = pool.kv_pools[0]
    assert torch.equal(key[0].transpose(0, 1), torch.cat([kp[2], kp[4]], 0))
    assert torch.equal(value[1].transpose(0, 1), torch.cat([vp[5], vp[0]], 0))


def test_gather_out_of_range_ids_read_the_null_block(native_lib, device):
    pool = PagedKVCachePool(1, 4, 16, 8, 128, torch.bfloat16, device)
    pool.storage.copy_(torch.randn(pool.storage.shape, device=device).to(torch.bfloat16))
    (key, value), = pool.gather_blocks(torch.tensor([[1, 4, -1]], device=device))
    (want_k, want_v), = pool.gather_blocks(torch.tensor([[1, 0, 0]], device=device))
    assert torch.equal(key, want_k) and torch.equal(value, want_v)


@pytest.mark.parametrize("layers,bs,heads,dim,dtype", [
    (33, 16, 8, 128, torch.bfloat16),  # two launches (32 layers per launch)
    (2, 2, 1, 6, torch.bfloat16),      # 24-byte blocks: 4-byte pieces, fewer than the workgroups per block
    (2, 1, 1, 3, torch.bfloat16),      # 6-byte blocks: 2-byte pieces
    (3, 3, 2, 5, torch.float32),       # 120-byte blocks: 4-byte pieces, one part each
    (2, 16, 4, 64, torch.float32),     # 16 KiB blocks
], ids=["33layers", "piece4", "piece2", "fp32odd", "fp32"])
def test_gather_block_shapes(native_lib, device, layers, bs, heads, dim, dtype):
    """Every block size the wide and narrow piece forms cover, against the closed form
    out[b, j] = pool[ids[b, j]] (ids outside the pool read block 0)."""
    gen = torch.Generator().manual_seed(layers * 100 + bs)
    nb = 12
    pool = PagedKVCachePool(layers, nb, bs, heads, dim, dtype, device)
    cpu = torch.randn(pool.storage.shape, generator=gen).to(dtype)
    pool.storage.copy_(cpu)
    ids = torch.tensor([[5, 11, 0, 3], [nb + 2, 7, -1, 7]])
    got = pool.gather_blocks(ids.to(device))
    fixed = ids.clamp(min=0).masked_fill(ids >= nb, 0)
    for layer, (gk, gv) in enumerate(got):
        for kv, g in ((0, gk), (1, gv)):
            want = cpu[layer, kv][fixed].reshape(2, 4 * bs, heads, dim).transpose(1, 2)
            assert_bit_equal(g.cpu(), want)


def test_gather_strided_block_ids(native_lib, device):
    """Block ids as a column slice of a packed metadata tensor (row stride != width)."""
    pool = PagedKVCachePool(1, 8, 16, 8, 128, torch.bfloat16, device)
    pool.storage.copy_(torch.randn(pool.storage.shape, device=device).to(torch.bfloat16))
    packed = torch.tensor([[9, 9, 2, 5], [9, 9, 7, 0]], device=device)
    (key, _), = pool.gather_blocks(packed[:, 2:])
    ref = pool.kv_pools[0][0][packed[:, 2:]].view(2, 32, 8, 128).transpose(1, 2)
    assert torch.equal(key, ref)
