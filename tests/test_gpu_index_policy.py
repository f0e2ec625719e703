"""One out-of-range rule for every entry point, on the GPU: a block id outside [0, num_blocks)
read through a table reads the null block 0 (bit-identical to the same call with 0 in its place),
a write to a slot or block outside the pool is skipped; with ``set_index_checks(True)`` every
entry point raises IndexError first, as the reference's tensor indexing does."""

import pytest
import torch

from mini_infra_qwen3_amd import data_plane

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


@pytest.fixture
def checks():
    previous = data_plane.set_index_checks(True)
    yield
    data_plane.set_index_checks(previous)


def pools(device, num_blocks=12, seed=0):
    g = torch.Generator(device=device).manual_seed(seed)
    return [torch.randn((num_blocks, 16, 8, 128), generator=g, device=device).to(torch.bfloat16) for _ in range(2)]


def bad_and_fixed(table, num_blocks):
    """The table with two entries inside every context replaced by ids outside the pool, and the
    same table with zeros there."""
    bad, fixed = table.clone(), table.clone()
    bad[:, 0], bad[:, 1] = num_blocks + 3, -2
    fixed[:, 0], fixed[:, 1] = 0, 0
    return bad, fixed


@pytest.mark.parametrize("exact", [False, True])
def test_decode_reads_block_zero(native_lib, device, exact):
    kp, vp = pools(device)
    q = torch.randn((3, 16, 128), device=device).to(torch.bfloat16)
    table = torch.tensor([[1, 2, 3, 4], [5, 6, 7, 0], [8, 9, 10, 11]], device=device)
    ctx = torch.tensor([60, 40, 64], device=device)
    bad, fixed = bad_and_fixed(table, kp.shape[0])
    got = data_plane.paged_decode_attention(q, kp, vp, bad, ctx, SCALE, exact=exact)
    want = data_plane.paged_decode_attention(q, kp, vp, fixed, ctx, SCALE, exact=exact)
    assert torch.equal(got, want)


@pytest.mark.parametrize("exact", [False, True])
def test_prefill_history_reads_block_zero(native_lib, device, exact):
    kp, vp = pools(device)
    q = torch.randn((2, 16, 40, 128), device=device).to(torch.bfloat16)
    k = torch.randn((2, 8, 40, 128), device=device).to(torch.bfloat16)
    v = torch.randn((2, 8, 40, 128), device=device).to(torch.bfloat16)
    hist = torch.tensor([[1, 2, 3], [4, 5, 6]], device=device)
    starts, lens = torch.tensor([48, 33], device=device), torch.tensor([40, 25], device=device)
    bad, fixed = bad_and_fixed(hist, kp.shape[0])
    got = data_plane.chunked_prefill_attention(q, k, v, kp, vp, bad, starts, lens, SCALE, exact=exact)
    want = data_plane.chunked_prefill_attention(q, k, v, kp, vp, fixed, starts, lens, SCALE, exact=exact)
    assert torch.equal(got, want)


@pytest.mark.parametrize("exact", [False, True])
def test_mixed_reads_block_zero_and_skips_bad_slots(native_lib, device, exact):
    kp, vp = pools(device, num_blocks=16)
    tokens = 20 + 2
    q = torch.randn((tokens, 16, 128), device=device).to(torch.bfloat16)
    k = torch.randn((tokens, 8, 128), device=device).to(torch.bfloat16)
    v = torch.randn((tokens, 8, 128), device=device).to(torch.bfloat16)
    hist = torch.tensor([[1, 2, 3]], device=device)
    starts, lens = torch.tensor([40], device=device), torch.tensor([20], device=device)
    dec = torch.tensor([[4, 5, 6], [7, 8, 9]], device=device)
    ctx = torch.tensor([40, 35], device=device)
    slots = torch.tensor([16 * 16 + 4, -7], device=device)  # both outside the pool: no write
    hbad, hfix = bad_and_fixed(hist, kp.shape[0])
    dbad, dfix = bad_and_fixed(dec, kp.shape[0])
    k1, v1, k2, v2 = kp.clone(), vp.clone(), kp.clone(), vp.clone()
    got = data_plane.mixed_paged_attention(q, k, v, k1, v1, 1, 20, hbad, starts, lens, dbad, ctx, slots, SCALE,
                                           exact=exact)
    want = data_plane.mixed_paged_attention(q, k, v, k2, v2, 1, 20, hfix, starts, lens, dfix, ctx, slots, SCALE,
                                            exact=exact)
    assert torch.equal(got, want)
    assert torch.equal(k1, kp) and torch.equal(v1, vp)


def test_gather_pack_read_block_zero_and_unpack_skips(native_lib, device):
    kp, vp = pools(device)
    ids = torch.tensor([[3, 40, -1]], device=device)
    outs = [torch.empty((1, 48, 8, 128), dtype=torch.bfloat16, device=device) for _ in range(2)]
    data_plane.gather_blocks([kp], [vp], ids, [outs[0]], [outs[1]])
    want = [torch.empty_like(outs[0]) for _ in range(2)]
    data_plane.gather_blocks([kp], [vp], torch.tensor([[3, 0, 0]], device=device), [want[0]], [want[1]])
    assert torch.equal(outs[0], want[0]) and torch.equal(outs[1], want[1])
    rec = data_plane.pack_blocks([kp], [vp], torch.tensor([40, 0], device=device))
    assert torch.equal(rec[0], rec[1])
    k1, v1 = kp.clone(), vp.clone()
    data_plane.unpack_blocks(rec, [k1], [v1], torch.tensor([12, -5], device=device))
    assert torch.equal(k1, kp) and torch.equal(v1, vp)


def test_scatter_skips_slots_outside_the_pool(native_lib, device):
    kp, vp = pools(device)
    src_k = torch.randn((1, 8, 3, 128), device=device).to(torch.bfloat16)
    src_v = torch.randn((1, 8, 3, 128), device=device).to(torch.bfloat16)
    k1, v1 = kp.clone(), vp.clone()
    slots = torch.tensor([5, 12 * 16, -3], device=device)
    data_plane.reshape_and_cache([src_k], [src_v], slots, [k1], [v1], torch.zeros(3, dtype=torch.long, device=device),
                                 torch.arange(3, device=device))
    want_k, want_v = kp.clone(), vp.clone()
    want_k.view(-1, 8, 128)[5] = src_k[0, :, 0]
    want_v.view(-1, 8, 128)[5] = src_v[0, :, 0]
    assert torch.equal(k1, want_k) and torch.equal(v1, want_v)


def test_checks_raise_like_the_reference(native_lib, device, checks):
    kp, vp = pools(device)
    q = torch.randn((1, 16, 128), device=device).to(torch.bfloat16)
    ctx = torch.tensor([20], device=device)
    with pytest.raises(IndexError):
        data_plane.paged_decode_attention(q, kp, vp, torch.tensor([[1, 12]], device=device), ctx, SCALE)
    with pytest.raises(IndexError):
        data_plane.paged_decode_attention(q, kp, vp, torch.tensor([[-1, 2]], device=device), ctx, SCALE, exact=True)
    data_plane.paged_decode_attention(q, kp, vp, torch.tensor([[11, 0]], device=device), ctx, SCALE)  # in range
    src = torch.randn((1, 8, 1, 128), device=device).to(torch.bfloat16)
    with pytest.raises(IndexError):
        data_plane.reshape_and_cache([src], [src], torch.tensor([12 * 16], device=device), [kp], [vp])
    data_plane.reshape_and_cache([src], [src], torch.tensor([-1], device=device), [kp], [vp])  # no-write marker
    outs = [torch.empty((1, 16, 8, 128), dtype=torch.bfloat16, device=device) for _ in range(2)]
    with pytest.raises(IndexError):
        data_plane.gather_blocks([kp], [vp], torch.tensor([[12]], device=device), [outs[0]], [outs[1]])
    with pytest.raises(IndexError):
        data_plane.pack_blocks([kp], [vp], torch.tensor([12], device=device))
    qh = torch.randn((1, 16, 8, 128), device=device).to(torch.bfloat16)
    kh = torch.randn((1, 8, 8, 128), device=device).to(torch.bfloat16)
    with pytest.raises(IndexError):
        data_plane.chunked_prefill_attention(qh, kh, kh, kp, vp, torch.tensor([[13]], device=device),
                                             torch.tensor([16], device=device), torch.tensor([8], device=device), SCALE)
    qm = torch.randn((9, 16, 128), device=device).to(torch.bfloat16)
    km = torch.randn((9, 8, 128), device=device).to(torch.bfloat16)
    with pytest.raises(IndexError):
        data_plane.mixed_paged_attention(qm, km, km, kp, vp, 1, 8, torch.zeros((1, 0), dtype=torch.long, device=device),
                                         torch.tensor([0], device=device), torch.tensor([8], device=device),
                                         torch.tensor([[2]], device=device), torch.tensor([5], device=device),
                                         torch.tensor([12 * 16], device=device), SCALE)
