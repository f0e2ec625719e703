"""mi_paged_decode_attention_noalloc (scratch in the library's fixed device array) against
mi_paged_decode_attention with a caller workspace, called through the C ABI: bit-identical
outputs on two calls in a row, the second smaller (the array keeps the first call's partials,
which the second must not read), on launches that take the block-range kernel and cut sequences
between ranges (so the scratch is used)."""

import ctypes

import pytest
import torch

from mini_infra_qwen3_amd import _native

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _case(seed, batch, lo, hi, num_blocks, device):
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=gen)
    need = (ctx + 15) // 16
    max_blocks = int(need.max())
    perm = torch.randperm(num_blocks - 1, generator=gen) + 1
    tables = torch.zeros(batch, max_blocks, dtype=torch.long)
    at = 0
    for b in range(batch):
        n = int(need[b])
        tables[b, :n] = perm[at:at + n]
        at += n
    assert at <= num_blocks - 1
    dgen = torch.Generator(device=device).manual_seed(seed)
    key_pool = torch.randn(num_blocks, 16, 8, 128, generator=dgen, device=device).to(torch.bfloat16)
    value_pool = torch.randn(num_blocks, 16, 8, 128, generator=dgen, device=device).to(torch.bfloat16)
    query = torch.randn(batch, 16, 128, generator=dgen, device=device).to(torch.bfloat16)
    return query, key_pool, value_pool, tables.to(device), ctx.to(device), max_blocks


def _call(lib, noalloc, query, key_pool, value_pool, tables, ctx, max_blocks):
    batch = query.shape[0]
    out = torch.full((batch, 16 * 128), float("nan"), dtype=torch.bfloat16, device=query.device)
    stream = torch.cuda.current_stream().cuda_stream
    args = (out.data_ptr(), out.stride(0), query.data_ptr(), query.stride(0), query.stride(1), key_pool.data_ptr(),
            value_pool.data_ptr(), key_pool.shape[0], tables.data_ptr(), tables.stride(0), max_blocks,
            ctx.data_ptr(), 1, batch, 16, 8, 128, 16, ctypes.c_float(SCALE))
    if noalloc:
        rc = lib.mi_paged_decode_attention_noalloc(*args, stream)
    else:
        need = lib.mi_paged_decode_workspace_bytes(batch, max_blocks, 16, 8, 128, 16)
        ws = torch.empty(need, dtype=torch.uint8, device=query.device)
        rc = lib.mi_paged_decode_attention(*args, ws.data_ptr(), need, stream)
    assert rc == _native.MI_OK, lib.mi_last_error()
    return out


def test_noalloc_matches_the_workspace_entry_point_on_two_calls(native_lib, device):
    lib = native_lib
    # batch 96 x 8 KV heads > 256 CUs: the block-range kernel; contexts up to 2600 tokens cut
    # sequences between ranges.  Then a smaller launch: fewer sequences, shorter contexts, fewer ranges.
    for seed, batch, lo, hi in [(0, 96, 300, 2600), (1, 40, 40, 700)]:
        print(f"[no-alloc] seed {seed} batch {batch} contexts U[{lo}, {hi}]", flush=True)
        case = _case(seed, batch, lo, hi, 12000, device)
        need = lib.mi_paged_decode_workspace_bytes(batch, case[-1], 16, 8, 128, 16)
        assert 0 < need <= (8 << 20)
        want = _call(lib, False, *case)
        got = _call(lib, True, *case)
        torch.cuda.synchronize()
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_small_launch_and_repeat(native_lib, device):
    """A launch the per-sequence kernel serves (no scratch), then the first case again: still exact."""
    lib = native_lib
    for seed, batch, lo, hi in [(2, 6, 1, 500), (0, 96, 300, 2600)]:
        case = _case(seed, batch, lo, hi, 12000, device)
        want = _call(lib, False, *case)
        got = _call(lib, True, *case)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
