"""Kernel 4, mixed form on the GPU: one launch serving a mixed step's chunk rows and decode rows
(``data_plane.mixed_paged_attention``).

* chunk rows: bit-identical to ``chunked_prefill_attention`` on the same rows (same kernel code);
* decode rows: within 2e-2 of the oracle's decode chain (gather + bias + attend) over the pool
  with the row's new token in its slot; with ``exact``, bit-identical to the exact decode kernel;
* the launch appends each decode row's K/V to its slot (rows with slot -1 or context 0 leave the
  pool untouched; context 0 gives a zero row), and nothing else in the pool changes.
"""

import pytest
import torch

from mini_infra_qwen3_amd import data_plane, workloads
from oracle import torch_ref

pytestmark = pytest.mark.gpu

TOL = 2e-2
SCALE = 128 ** -0.5


def make_case(seed, starts, lens, width, contexts, group=2, kv_heads=8, no_slot=(), block_size=16):
    """Pools with the chunk rows' histories and the decode rows' contexts (minus their new token)
    in permuted blocks; token-major q / k / v of the T = P width + D tokens."""
    gen = torch.Generator().manual_seed(seed)
    rows, decode_rows = len(lens), len(contexts)
    totals = list(starts) + list(contexts)
    num_blocks = 1 + sum(-(-t // block_size) for t in totals) + 3
    tables = workloads.permuted_tables(totals, num_blocks, gen, block_size=block_size)
    kp = torch.randn(num_blocks, block_size, kv_heads, 128, generator=gen).to(torch.bfloat16)
    vp = torch.randn(num_blocks, block_size, kv_heads, 128, generator=gen).to(torch.bfloat16)
    tokens = rows * width + decode_rows
    q = torch.randn(tokens, group * kv_heads, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(tokens, kv_heads, 128, generator=gen).to(torch.bfloat16)
    v = torch.randn(tokens, kv_heads, 128, generator=gen).to(torch.bfloat16)
    nb = max([-(-s // block_size) for s in starts], default=0)
    hist = torch.zeros((rows, nb), dtype=torch.long)
    for b, s in enumerate(starts):
        hist[b, :-(-s // block_size)] = torch.tensor(tables[b][:-(-s // block_size)], dtype=torch.long)
    mb = max([-(-c // block_size) for c in contexts], default=0)
    dec = torch.zeros((decode_rows, max(mb, 1)), dtype=torch.long)
    slots = torch.full((decode_rows,), -1, dtype=torch.long)
    for d, c in enumerate(contexts):
        t = tables[rows + d]
        dec[d, :len(t)] = torch.tensor(t, dtype=torch.long)
        if c > 0 and d not in no_slot:
            slots[d] = t[(c - 1) // block_size] * block_size + (c - 1) % block_size
    return dict(q=q, k=k, v=v, kp=kp, vp=vp, hist=hist, starts=torch.tensor(starts, dtype=torch.long),
                lens=torch.tensor(lens, dtype=torch.long), dec=dec, ctx=torch.tensor(contexts, dtype=torch.long),
                slots=slots, rows=rows, width=width, tables=tables)


def run_mixed(case, device, exact=False):
    c = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in case.items()}
    kp, vp = c["kp"].clone(), c["vp"].clone()
    out = data_plane.mixed_paged_attention(c["q"], c["k"], c["v"], kp, vp, c["rows"], c["width"], c["hist"],
                                           c["starts"], c["lens"], c["dec"], c["ctx"], c["slots"], SCALE,
                                           exact=exact)
    return out, kp, vp


def pool_with_new_tokens(case, only_slots):
    """The pool with each decode row's new K/V at its context's last position (only at the rows'
    slots when ``only_slots``)."""
    kp, vp = case["kp"].clone(), case["vp"].clone()
    n = case["rows"] * case["width"]
    bs = kp.shape[1]
    for d, c in enumerate(case["ctx"].tolist()):
        if c <= 0 or (only_slots and case["slots"][d] < 0):
            continue
        block = case["dec"][d, (c - 1) // bs]
        kp[block, (c - 1) % bs] = case["k"][n + d]
        vp[block, (c - 1) % bs] = case["v"][n + d]
    return kp, vp


def chunk_rows_apart(case, device, exact=False):
    rows, width = case["rows"], case["width"]
    n = rows * width
    heads, kv_heads = case["q"].shape[1], case["k"].shape[1]
    q = case["q"][:n].view(rows, width, heads, 128).transpose(1, 2)
    k = case["k"][:n].view(rows, width, kv_heads, 128).transpose(1, 2)
    v = case["v"][:n].view(rows, width, kv_heads, 128).transpose(1, 2)
    out = data_plane.chunked_prefill_attention(q.to(device), k.to(device), v.to(device), case["kp"].to(device),
                                               case["vp"].to(device), case["hist"].to(device),
                                               case["starts"].to(device), case["lens"].to(device), SCALE,
                                               exact=exact)
    return out.reshape(n, -1)


CASES = [
    # (starts, lens, width, contexts)
    ([0, 40], [37, 64], 64, [1, 17, 300, 0, 64]),     # chunk without / with history; decode edges and a pad row
    ([130], [1], 1, [33, 2000]),                        # a 1-token chunk, a long decode context
    ([16, 0, 513], [200, 129, 70], 200, [5]),           # three chunk rows, one decode row
    ([], [], 0, [9, 100, 16, 0]),                        # decode rows only
    ([70], [130], 130, []),                              # chunk rows only
]


@pytest.mark.parametrize("starts,lens,width,contexts", CASES)
def test_mixed_matches_the_two_paths(native_lib, device, starts, lens, width, contexts):
    case = make_case(len(contexts) + sum(lens), starts, lens, width, contexts)
    out, kp, vp = run_mixed(case, device)
    out = out.cpu()
    n = case["rows"] * case["width"]
    if n:
        assert torch.equal(out[:n], chunk_rows_apart(case, device).cpu())
    want_kp, want_vp = pool_with_new_tokens(case, only_slots=True)
    assert torch.equal(kp.cpu(), want_kp) and torch.equal(vp.cpu(), want_vp)
    if contexts:
        akp, avp = pool_with_new_tokens(case, only_slots=False)
        heads = case["q"].shape[1]
        ref = torch_ref.paged_decode_attention(case["q"][n:], akp, avp, case["dec"], case["ctx"], SCALE)
        got = out[n:].float()
        for d, c in enumerate(contexts):
            if c == 0:
                assert not got[d].any(), f"decode row {d}: context 0 must give a zero row"
            else:
                err = (got[d] - ref[d].float()).abs().max().item()
                assert err <= TOL, f"decode row {d} (context {c}): max-abs {err}"
        assert got.shape == (len(contexts), heads * 128)


@pytest.mark.parametrize("group,kv_heads", [(1, 8), (4, 8), (5, 4), (8, 2)])
def test_mixed_other_gqa_groups(native_lib, device, group, kv_heads):
    starts, lens, width, contexts = [20, 0], [45, 33], 48, [7, 150, 0]
    case = make_case(group * 10 + kv_heads, starts, lens, width, contexts, group=group, kv_heads=kv_heads)
    out, kp, vp = run_mixed(case, device)
    out = out.cpu()
    n = case["rows"] * width
    assert torch.equal(out[:n], chunk_rows_apart(case, device).cpu())
    akp, avp = pool_with_new_tokens(case, only_slots=False)
    ref = torch_ref.paged_decode_attention(case["q"][n:], akp, avp, case["dec"], case["ctx"], SCALE)
    for d, c in enumerate(contexts):
        got = out[n + d].float()
        if c == 0:
            assert not got.any()
        else:
            assert (got - ref[d].float()).abs().max().item() <= TOL


def test_mixed_row_without_slot_attends_its_own_token(native_lib, device):
    """A decode row with slot -1 still sees its new token (read from k / v, not the pool) and
    leaves the pool as it was."""
    case = make_case(5, [8], [20], 20, [40, 41], no_slot=(1,))
    out, kp, vp = run_mixed(case, device)
    n = 20
    want_kp, want_vp = pool_with_new_tokens(case, only_slots=True)
    assert torch.equal(kp.cpu(), want_kp) and torch.equal(vp.cpu(), want_vp)
    akp, avp = pool_with_new_tokens(case, only_slots=False)
    ref = torch_ref.paged_decode_attention(case["q"][n:], akp, avp, case["dec"], case["ctx"], SCALE)
    assert (out.cpu()[n:].float() - ref.float()).abs().max().item() <= TOL


def test_mixed_pools_of_32_token_blocks(native_lib, device):
    case = make_case(11, [50], [40], 40, [31, 90, 1], block_size=32)
    out, kp, vp = run_mixed(case, device)
    n = 40
    want_kp, want_vp = pool_with_new_tokens(case, only_slots=True)
    assert torch.equal(kp.cpu(), want_kp) and torch.equal(vp.cpu(), want_vp)
    akp, avp = pool_with_new_tokens(case, only_slots=False)
    ref = torch_ref.paged_decode_attention(case["q"][n:], akp, avp, case["dec"], case["ctx"], SCALE)
    assert (out.cpu()[n:].float() - ref.float()).abs().max().item() <= TOL
    ref_chunk = torch_ref.chunked_prefill_attention(
        case["q"][:n].view(1, n, 16, 128).transpose(1, 2), case["k"][:n].view(1, n, 8, 128).transpose(1, 2),
        case["v"][:n].view(1, n, 8, 128).transpose(1, 2), (case["kp"], case["vp"]), case["hist"], [50], [40], SCALE)
    assert (out.cpu()[:n].float() - ref_chunk[0].reshape(n, -1).float()).abs().max().item() <= TOL


@pytest.mark.parametrize("starts,lens,width,contexts", CASES[:4])
def test_mixed_exact_is_bit_identical_to_the_exact_kernels(native_lib, device, starts, lens, width, contexts):
    case = make_case(100 + len(contexts), starts, lens, width, contexts)
    out, kp, vp = run_mixed(case, device, exact=True)
    out = out.cpu()
    n = case["rows"] * case["width"]
    if n:
        assert torch.equal(out[:n], chunk_rows_apart(case, device, exact=True).cpu())
    want_kp, want_vp = pool_with_new_tokens(case, only_slots=True)
    assert torch.equal(kp.cpu(), want_kp) and torch.equal(vp.cpu(), want_vp)
    akp, avp = pool_with_new_tokens(case, only_slots=False)
    apart = data_plane.paged_decode_attention(case["q"][n:].to(device), akp.to(device), avp.to(device),
                                              case["dec"].to(device), case["ctx"].to(device), SCALE, exact=True)
    assert torch.equal(out[n:], apart.cpu())
    ref = torch_ref.paged_decode_attention(case["q"][n:], akp, avp, case["dec"], case["ctx"], SCALE, exact=True)
    assert (out[n:].float() - ref.float()).abs().max().item() <= 4e-3


def ragged_of(case, tail=3, gap=0):
    """The case with its chunk rows packed in order (each row's real tokens, no padding), ``gap`` pad
    tokens before each row and ``tail`` after the last, then the decode tokens: (q, k, v,
    chunk_first, chunk_tokens, keep, real) -- ``keep[j]`` is the padded-layout token of ragged
    token ``real[j]``; every other ragged chunk token is a pad token."""
    rows, width = case["rows"], case["width"]
    n = rows * width
    order, first = [], []  # padded-layout token of each ragged chunk token, -1 for a pad token
    for b, l in enumerate(case["lens"].tolist()):
        order += [-1] * gap
        first.append(len(order))
        order += [b * width + i for i in range(width - l, width)]
    order += [-1] * tail
    idx = torch.tensor([i if i >= 0 else n + j for j, i in enumerate(order)], dtype=torch.long)
    gen = torch.Generator().manual_seed(99)
    parts = []
    for name in ("q", "k", "v"):
        t = case[name]
        pads = torch.randn((len(order),) + tuple(t.shape[1:]), generator=gen).to(t.dtype)
        parts.append(torch.cat((torch.cat((t[:n], pads))[idx], t[n:])))
    real = [j for j, i in enumerate(order) if i >= 0]
    keep = [i for i in order if i >= 0]
    return parts[0], parts[1], parts[2], torch.tensor(first, dtype=torch.long), len(order), keep, real


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("starts,lens,width,contexts", [c for c in CASES if c[0]])
@pytest.mark.parametrize("tail,gap", [(3, 0), (0, 0), (5, 2)])
def test_mixed_ragged_rows_give_the_padded_rows_bits(native_lib, device, exact, starts, lens, width, contexts, tail,
                                                      gap):
    """Ragged chunk rows (chunk_first / chunk_tokens: each row's real tokens packed in order, pad
    tokens before the rows and after them) give, bit for bit, the outputs of the same rows
    left-padded to the width, the same decode rows and the same pool appends; every pad token gets
    a zero row (over a sentinel-filled ``out``)."""
    case = make_case(17, starts, lens, width, contexts)
    want, want_kp, want_vp = run_mixed(case, device, exact=exact)
    q, k, v, first, chunk_tokens, keep, real = ragged_of(case, tail, gap)
    c = {key: (val.to(device) if torch.is_tensor(val) else val) for key, val in case.items()}
    kp, vp = c["kp"].clone(), c["vp"].clone()
    out = torch.full((q.shape[0], q.shape[1] * 128), -7.5, dtype=torch.bfloat16, device=device)
    data_plane.mixed_paged_attention(q.to(device), k.to(device), v.to(device), kp, vp, c["rows"], c["width"],
                                     c["hist"], c["starts"], c["lens"], c["dec"], c["ctx"], c["slots"], SCALE,
                                     out=out, exact=exact, chunk_first=first.to(device), chunk_tokens=chunk_tokens)
    torch.cuda.synchronize()
    n = case["rows"] * case["width"]
    pad = sorted(set(range(chunk_tokens)) - set(real))
    assert torch.equal(out[real], want[keep])
    assert len(pad) == tail + gap * case["rows"] and not out[pad].any()  # pad tokens: zero rows
    assert torch.equal(out[chunk_tokens:], want[n:])                       # decode rows
    assert torch.equal(kp, want_kp) and torch.equal(vp, want_vp)


@pytest.mark.parametrize("exact", [False, True])
def test_ragged_tokens_without_chunk_rows_get_zero_rows_through_the_c_abi(native_lib, device, exact):
    """Ragged chunk tokens with no chunk row (``chunk_first`` set, P = 0, C = 5): the entry point
    writes zero rows for all C tokens and serves the decode rows after them with the bits (and pool
    appends) of the same rows without chunk tokens.  Called through the C ABI: the Python wrapper
    refuses this form."""
    case = make_case(5, [], [], 0, [9, 100, 16, 0])
    want, want_kp, want_vp = run_mixed(case, device, exact=exact)
    chunk_tokens = 5
    gen = torch.Generator().manual_seed(3)
    c = {key: (val.to(device) if torch.is_tensor(val) else val) for key, val in case.items()}
    q, k, v = (torch.cat((torch.randn((chunk_tokens,) + tuple(c[n].shape[1:]), generator=gen).to(torch.bfloat16)
                          .to(device), c[n])) for n in ("q", "k", "v"))
    kp, vp = c["kp"].clone(), c["vp"].clone()
    out = torch.full((q.shape[0], q.shape[1] * 128), -7.5, dtype=torch.bfloat16, device=device)
    first = torch.zeros(1, dtype=torch.long, device=device)  # never read: no chunk row
    entry = native_lib.mi_mixed_paged_attention_exact if exact else native_lib.mi_mixed_paged_attention
    rc = entry(out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
               k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), kp.data_ptr(), vp.data_ptr(), kp.shape[0],
               0, 0, chunk_tokens, first.data_ptr(), None, 0, 0, None, None, 1,
               c["ctx"].shape[0], c["dec"].data_ptr(), c["dec"].stride(0), c["dec"].shape[1], c["ctx"].data_ptr(), 1,
               c["slots"].data_ptr(), 1, q.shape[1], k.shape[1], 128, 16, SCALE,
               torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, native_lib.mi_last_error()
    assert not out[:chunk_tokens].any()
    assert torch.equal(out[chunk_tokens:], want)
    assert torch.equal(kp, want_kp) and torch.equal(vp, want_vp)


def test_mixed_rejects_bad_shapes(native_lib, device):
    case = make_case(3, [0], [10], 10, [5])
    c = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in case.items()}
    with pytest.raises(ValueError):  # token count is not P L + D
        data_plane.mixed_paged_attention(c["q"][:-1], c["k"][:-1], c["v"][:-1], c["kp"], c["vp"], 1, 10, c["hist"],
                                         c["starts"], c["lens"], c["dec"], c["ctx"], c["slots"], SCALE)
    with pytest.raises(ValueError):  # one slot per decode row
        data_plane.mixed_paged_attention(c["q"], c["k"], c["v"], c["kp"], c["vp"], 1, 10, c["hist"], c["starts"],
                                         c["lens"], c["dec"], c["ctx"], c["slots"][:0], SCALE)
    with pytest.raises(ValueError):  # ragged chunk tokens but no chunk row
        data_plane.mixed_paged_attention(c["q"], c["k"], c["v"], c["kp"], c["vp"], 0, 10, c["hist"][:0],
                                         c["starts"][:0], c["lens"][:0], c["dec"], c["ctx"], c["slots"], SCALE,
                                         chunk_first=c["starts"][:0], chunk_tokens=10)
