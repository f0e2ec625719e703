"""Pins the oracle (CPU restatement of the reference torch path) before the GPU tests compare
against it: against the reference suite's known-answer tests, the closed forms of
``oracle.closed_form`` (numpy indexing, fp64 loops) and the reference's own invariants."""

import numpy as np
import pytest
import torch

from oracle import closed_form, torch_ref

HQ, HKV, D, BS = 16, 8, 128, 16
SCALE = D ** -0.5


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy()


def random_tables(gen: torch.Generator, ctx: list[int], num_blocks: int, bs: int = BS):
    need = [-(-c // bs) for c in ctx]
    perm = torch.randperm(num_blocks - 1, generator=gen)[: sum(need)] + 1
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n].tolist())
        k += n
    width = max(need)
    padded = torch.zeros((len(ctx), width), dtype=torch.long)
    for b, t in enumerate(tables):
        padded[b, :len(t)] = torch.tensor(t)
    return tables, padded


# ------------------------------------------------------------------ scatter / gather
def test_write_prefill_matches_closed_form_bit_exact():
    gen = torch.Generator().manual_seed(1)
    pools = torch_ref.make_pools(2, 12, 4, 2, 8)
    for k, v in pools:  # non-zero background: untouched rows must stay as they were
        k.copy_(torch.randn(k.shape, generator=gen).to(k.dtype))
        v.copy_(torch.randn(v.shape, generator=gen).to(v.dtype))
    before = [(bits(k), bits(v)) for k, v in pools]
    # K contiguous [B, H, L, D]; V a transpose view of [B, L, H, D] as the reference's v_proj gives
    cache = [(torch.randn(3, 2, 5, 8, generator=gen).to(torch.bfloat16),
              torch.randn(3, 5, 2, 8, generator=gen).to(torch.bfloat16).transpose(1, 2)) for _ in range(2)]
    rows = torch.tensor([0, 0, 1, 2, 2, 2])
    pos = torch.tensor([3, 4, 4, 1, 2, 4])
    slots = torch.tensor([17, 5, 40, 2, 33, 46])
    torch_ref.write_prefill(pools, cache, rows, pos, slots)
    for (k, v), (k0, v0), (ck, cv) in zip(pools, before, cache):
        assert np.array_equal(bits(k), closed_form.scatter_rows(k0, bits(ck), rows, pos, slots))
        assert np.array_equal(bits(v), closed_form.scatter_rows(v0, bits(cv), rows, pos, slots))


def test_write_prefill_arange_known_answer():
    """verification/smoke.py:299-318: arange K (+1000 per layer), V = K + 500, 6 tokens, block 4."""
    heads, dim, bs = 2, 4, 4
    pools = torch_ref.make_pools(2, 4, bs, heads, dim, dtype=torch.float32)
    layers = []
    for layer in range(2):
        key = torch.arange(heads * 6 * dim, dtype=torch.float32).view(1, heads, 6, dim) + layer * 1000.0
        layers.append((key, key + 500.0))
    table = [1, 2]
    rows, positions, slots = torch_ref.store_prefill_indices([table], [6], [0], 6, bs)
    torch_ref.write_prefill(pools, layers, torch.tensor(rows), torch.tensor(positions), torch.tensor(slots))
    for (kp, vp), (ek, ev) in zip(pools, layers):
        got_k = torch.cat([kp[b] for b in table], 0)[:6].transpose(0, 1).unsqueeze(0)
        got_v = torch.cat([vp[b] for b in table], 0)[:6].transpose(0, 1).unsqueeze(0)
        assert torch.equal(got_k, ek) and torch.equal(got_v, ev)
    assert not pools[0][0][0].any() and not pools[0][0][3].any()  # null block and free block untouched


def test_gather_blocks_arange_known_answer():
    """tests/unit/test_paged_kv_cache.py:265-280."""
    pools = torch_ref.make_pools(2, 6, 4, 2, 4, dtype=torch.float32)
    for k, v in pools:
        k.copy_(torch.arange(k.numel(), dtype=torch.float32).view_as(k))
        v.copy_(k + 0.5)
    ids = torch.tensor([[2, 4], [5, 0]])
    (key, value), _ = torch_ref.gather_blocks(pools, ids)
    assert tuple(key.shape) == (2, 2, 8, 4)
    kp, vp = pools[0]
    assert torch.equal(key[0].transpose(0, 1), torch.cat([kp[2], kp[4]], 0))
    assert torch.equal(value[1].transpose(0, 1), torch.cat([vp[5], vp[0]], 0))


def test_gather_blocks_matches_closed_form():
    gen = torch.Generator().manual_seed(2)
    pools = torch_ref.make_pools(1, 9, BS, HKV, D)
    pools[0][0].copy_(torch.randn(pools[0][0].shape, generator=gen).to(torch.bfloat16))
    ids = torch.tensor([[3, 0, 8], [1, 1, 7]])
    (key, _), = torch_ref.gather_blocks(pools, ids)
    expect = closed_form.gather_rows(bits(pools[0][0]), ids.numpy())
    assert np.array_equal(bits(key.transpose(1, 2)), expect)


# ---------------------------------------------------------------------- decode attention
def decode_case(seed: int, ctx: list[int], dtype=torch.float32, num_blocks: int = 64):
    gen = torch.Generator().manual_seed(seed)
    (key_pool, value_pool), = torch_ref.make_pools(1, num_blocks, BS, HKV, D, dtype=dtype)
    key_pool.copy_(torch.randn(key_pool.shape, generator=gen).to(dtype))
    value_pool.copy_(torch.randn(value_pool.shape, generator=gen).to(dtype))
    query = torch.randn(len(ctx), HQ, D, generator=gen).to(dtype)
    _, tables = random_tables(gen, ctx, num_blocks)
    return query, key_pool, value_pool, tables, torch.tensor(ctx)


@pytest.mark.parametrize("ctx", [[1, 16, 17], [40, 3, 33], [64, 5]])
def test_decode_oracle_fp32_matches_fp64_textbook(ctx):
    """Head mapping h // 2, masking t < ctx and the scale all agree with explicit fp64 loops."""
    q, kp, vp, tables, lens = decode_case(3, ctx)
    got = torch_ref.paged_decode_attention(q, kp, vp, tables, lens, SCALE).view(len(ctx), HQ, D)
    ref = closed_form.decode_attention_fp64(q.numpy(), kp.numpy(), vp.numpy(), tables.numpy(), lens.numpy(), SCALE)
    assert np.abs(got.numpy() - ref).max() < 1e-5


def test_decode_oracle_bf16_within_rounding_of_fp64():
    q, kp, vp, tables, lens = decode_case(4, [37, 64, 9, 50], dtype=torch.bfloat16)
    got = torch_ref.paged_decode_attention(q, kp, vp, tables, lens, SCALE).float().view(4, HQ, D)
    ref = closed_form.decode_attention_fp64(q.float().numpy(), kp.float().numpy(), vp.float().numpy(),
                                           tables.numpy(), lens.numpy(), SCALE)
    assert np.abs(got.numpy() - ref).max() < 2e-2


def test_decode_oracle_paged_equals_dense_per_request():
    """Reference invariant (tests/unit/test_paged_kv_cache.py:109-163): attention through the
    block table equals attention over each request's contiguous K/V."""
    ctx = [23, 7, 48]
    q, kp, vp, tables, lens = decode_case(5, ctx)
    paged = torch_ref.paged_decode_attention(q, kp, vp, tables, lens, SCALE)
    for b, n in enumerate(ctx):
        blocks = tables[b, : -(-n // BS)]
        k = kp[blocks].reshape(-1, HKV, D)[:n].transpose(0, 1).unsqueeze(0)
        v = vp[blocks].reshape(-1, HKV, D)[:n].transpose(0, 1).unsqueeze(0)
        dense = torch_ref.attend(q[b].view(1, HQ, 1, D), k, v, torch.zeros(1, 1, 1, n), SCALE)
        assert (paged[b] - dense.view(-1)).abs().max() < 1e-5


def test_decode_oracle_ignores_stale_tails_and_padding():
    """Reference invariant (tests/unit/test_paged_kv_cache.py:166-207): data past the context
    (stale tails of recycled blocks, null-padded entries) cannot change the output."""
    ctx = [5, 33]
    q, kp, vp, tables, lens = decode_case(6, ctx, dtype=torch.bfloat16)
    before = torch_ref.paged_decode_attention(q, kp, vp, tables, lens, SCALE)
    kp2, vp2 = kp.clone(), vp.clone()
    for b, n in enumerate(ctx):
        last = int(tables[b, (n - 1) // BS])
        kp2[last, (n - 1) % BS + 1:] = 77.0
        vp2[last, (n - 1) % BS + 1:] = -91.0
    kp2[0] = 55.0  # null block used by the padding of row 0
    vp2[0] = 13.0
    after = torch_ref.paged_decode_attention(q, kp2, vp2, tables, lens, SCALE)
    assert torch.equal(before, after)


def test_decode_step_appends_before_attending():
    """qwen3.py:282-292: the new token is written to its slot first and is part of the context."""
    ctx = [9, 16]
    q, kp, vp, tables, lens = decode_case(7, ctx, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(8)
    new_k = torch.randn(2, HKV, 1, D, generator=gen).to(torch.bfloat16)
    new_v = torch.randn(2, HKV, 1, D, generator=gen).to(torch.bfloat16)
    slots = torch.tensor([closed_form.slot_of(tables[b], n - 1, BS) for b, n in enumerate(ctx)])
    out = torch_ref.paged_decode_step(q.unsqueeze(2), new_k, new_v, (kp, vp), slots, tables, lens, SCALE)
    for b, n in enumerate(ctx):
        row = kp.view(-1, HKV, D)[slots[b]]
        assert torch.equal(row, new_k[b, :, 0])
    ref = torch_ref.paged_decode_attention(q, kp, vp, tables, lens, SCALE)
    assert torch.equal(out.view(2, -1), ref)


# ----------------------------------------------------------------- chunked prefill attention
def prefill_case(seed, starts, lens, dtype=torch.float32, num_blocks=32, bs=BS):
    gen = torch.Generator().manual_seed(seed)
    (kp, vp), = torch_ref.make_pools(1, num_blocks, bs, HKV, D, dtype=dtype)
    kp.copy_(torch.randn(kp.shape, generator=gen).to(dtype))
    vp.copy_(torch.randn(vp.shape, generator=gen).to(dtype))
    width = max(lens)
    q = torch.randn(len(lens), HQ, width, D, generator=gen).to(dtype)
    ck = torch.randn(len(lens), HKV, width, D, generator=gen).to(dtype)
    cv = torch.randn(len(lens), HKV, width, D, generator=gen).to(dtype)
    _, tables = random_tables(gen, [s + n for s, n in zip(starts, lens)], num_blocks, bs)
    nb = max(-(-s // bs) for s in starts)
    hist = torch.zeros((len(lens), nb), dtype=torch.long)
    for b, s in enumerate(starts):
        h = -(-s // bs)
        hist[b, :h] = tables[b, :h]
    return q, ck, cv, (kp, vp), hist


@pytest.mark.parametrize("starts,lens", [([0, 0], [5, 3]), ([20, 3], [7, 4]), ([32, 17, 1], [1, 6, 9])])
def test_chunked_prefill_oracle_matches_fp64_textbook(starts, lens):
    q, ck, cv, pool, hist = prefill_case(9, starts, lens)
    got = torch_ref.chunked_prefill_attention(q, ck, cv, pool, hist, starts, lens, SCALE)
    width = max(lens)
    nb = hist.shape[1]
    for b, (start, n) in enumerate(zip(starts, lens)):
        hk = pool[0][hist[b]].reshape(-1, HKV, D).transpose(0, 1).numpy() if nb else np.zeros((HKV, 0, D))
        hv = pool[1][hist[b]].reshape(-1, HKV, D).transpose(0, 1).numpy() if nb else np.zeros((HKV, 0, D))
        keys = np.concatenate([hk, ck[b].numpy()], axis=1)
        values = np.concatenate([hv, cv[b].numpy()], axis=1)
        h_len = nb * BS
        visible = np.zeros((width, h_len + width), dtype=bool)
        for i in range(width):
            visible[i, :min(start, h_len)] = True
            for j in range(width - n, i + 1):
                visible[i, h_len + j] = True
        ref = closed_form.prefill_attention_fp64(q[b].numpy(), keys, values, visible, SCALE)
        out = got[b].view(width, HQ, D).transpose(0, 1).numpy()
        valid = slice(width - n, width)  # left-padding rows are not compared
        assert np.abs(out[:, valid] - ref[:, valid]).max() < 1e-5
