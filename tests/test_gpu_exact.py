"""Reference-numerics kernels on the GPU (mi_paged_decode_attention_exact,
mi_chunked_prefill_attention_exact, the exact RMSNorm of mi_rms_norm / mi_qk_norm_rope) against the
oracle's definitions (torch_ref.attend_exact, rms_norm_exact): bit for bit, with the oracle run
both on the CPU and on cuda:0.  Also within a few bf16 ulps of the op-for-op restatement of the
reference (torch_ref.attend), which sums in ATen's order.  Covers every GQA group, contexts past
the LDS score cache (the recompute passes), the fused prologue with its K/V append, chunked prefill
with history, ragged rows and left padding (zero rows)."""

import pytest
import torch

from mini_infra_qwen3_amd import data_plane, workloads
from oracle import torch_ref

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5
NEAR = 4e-3  # exact vs the op-for-op oracle: a few bf16 ulps of |out| < 1


def assert_bits(got, want):
    g, w = got.cpu().view(torch.int16), want.cpu().view(torch.int16)
    assert torch.equal(g, w), f"{(g != w).sum().item()} of {g.numel()} values differ"


def decode_case(seed, batch, lo, hi, kv_heads, group, num_blocks):
    gen = torch.Generator().manual_seed(seed)
    ctx = workloads.uniform_lengths(batch, lo, hi, gen)
    tables = workloads.permuted_tables(ctx, num_blocks, gen)
    bt = workloads.padded(tables)
    kp = torch.randn(num_blocks, 16, kv_heads, 128, generator=gen).bfloat16()
    vp = torch.randn(num_blocks, 16, kv_heads, 128, generator=gen).bfloat16()
    q = torch.randn(batch, kv_heads * group, 128, generator=gen).bfloat16()
    return q, kp, vp, bt, torch.tensor(ctx)


@pytest.mark.parametrize("seed,batch,lo,hi,kv_heads,group,num_blocks", [
    (0, 8, 64, 512, 8, 2, 4096),     # the one-layer decode step's shape (batch 8, contexts U[64, 512])
    (1, 5, 1, 40, 8, 2, 64),         # contexts of one token and partial blocks
    (2, 3, 100, 700, 4, 4, 400),
    (3, 2, 9000, 9700, 2, 8, 1300),  # past the LDS score cache: scores recomputed per pass
    (4, 4, 30, 300, 8, 5, 200),
    (5, 3, 50, 300, 8, 1, 200),
    (6, 40, 200, 1200, 8, 2, 4000),  # a decode batch of the continuous-batching run's size
])
def test_exact_decode_is_bit_identical_to_the_oracle(device, seed, batch, lo, hi, kv_heads, group, num_blocks):
    q, kp, vp, bt, ctx = decode_case(seed, batch, lo, hi, kv_heads, group, num_blocks)
    got = data_plane.paged_decode_attention(q.to(device), kp.to(device), vp.to(device), bt.to(device),
                                            ctx.to(device), SCALE, exact=True)
    want_gpu = torch_ref.paged_decode_attention(q.to(device), kp.to(device), vp.to(device), bt.to(device),
                                                ctx.to(device), SCALE, exact=True)
    want_cpu = torch_ref.paged_decode_attention(q, kp, vp, bt, ctx, SCALE, exact=True)
    assert_bits(got, want_gpu)
    assert_bits(got, want_cpu)
    ref = torch_ref.paged_decode_attention(q, kp, vp, bt, ctx, SCALE)
    assert (got.float().cpu() - ref.float()).abs().max().item() <= NEAR


def test_exact_decode_empty_context_and_null_padding(device):
    """Context 0 gives a zero row; table entries past the context (null block 0, stale ids) are never read."""
    q, kp, vp, bt, ctx = decode_case(9, 4, 20, 60, 8, 2, 64)
    ctx[1] = 0
    bt = torch.cat((bt, torch.full((4, 3), 7, dtype=torch.long)), dim=1)  # stale ids past every context
    got = data_plane.paged_decode_attention(q.to(device), kp.to(device), vp.to(device), bt.to(device),
                                            ctx.to(device), SCALE, exact=True)
    assert not got[1].any()
    want = torch_ref.paged_decode_attention(q, kp, vp, bt, ctx, SCALE, exact=True)
    assert_bits(got, want)


def test_exact_decode_plain_form_ignores_slot_mapping(device):
    """Without the prologue (q_weight NULL) k, v and slot_mapping are ignored: a C caller that
    passes real slots with NULL k / v gets the plain attention and an unchanged pool."""
    from mini_infra_qwen3_amd import _native

    q, kp, vp, bt, ctx = decode_case(12, 4, 20, 60, 8, 2, 64)
    q, kpd, vpd, bt, ctx = q.to(device), kp.to(device), vp.to(device), bt.to(device), ctx.to(device)
    slots = (bt[:, 0] * 16 + 3).contiguous()
    out = torch.empty(4, 16 * 128, dtype=torch.bfloat16, device=device)
    lib = _native.load()
    rc = lib.mi_paged_decode_attention_exact(
        out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), q.stride(1), None, 0, None, 0, None, None, None,
        None, 0.0, slots.data_ptr(), 1, kpd.data_ptr(), vpd.data_ptr(), kp.shape[0], bt.data_ptr(), bt.stride(0),
        bt.shape[1], ctx.data_ptr(), 1, 4, 16, 8, 128, 16, SCALE, None, 0, data_plane._stream(device))
    _native.check(rc, "mi_paged_decode_attention_exact")
    torch.cuda.synchronize()
    assert_bits(kpd, kp)
    assert_bits(vpd, vp)
    assert_bits(out, torch_ref.paged_decode_attention(q.cpu(), kp, vp, bt.cpu(), ctx.cpu(), SCALE, exact=True))


def test_exact_decode_prologue_padding_row_appends_nothing(device):
    """Prologue form: a row of context 0 (a padding row) gets a zero output and appends nothing,
    even with a slot inside the pool; the other rows append as usual."""
    gen = torch.Generator().manual_seed(21)
    batch, nb = 3, 32
    kp = torch.randn(nb, 16, 8, 128, generator=gen).bfloat16()
    vp = torch.randn(nb, 16, 8, 128, generator=gen).bfloat16()
    q_raw = torch.randn(batch, 16 * 128, generator=gen).bfloat16()
    k_raw = torch.randn(batch, 8 * 128, generator=gen).bfloat16()
    v_raw = torch.randn(batch, 8 * 128, generator=gen).bfloat16()
    weight = torch.ones(128).bfloat16()
    cos, sin = torch.ones(batch, 128).bfloat16(), torch.zeros(batch, 128).bfloat16()
    bt = torch.tensor([[3, 4], [5, 0], [6, 7]])
    ctx = torch.tensor([20, 0, 17])
    slots = torch.tensor([4 * 16 + 3, 5 * 16 + 9, 7 * 16 + 0])
    kpd, vpd = kp.to(device), vp.to(device)
    got = data_plane.paged_decode_attention_fused(
        q_raw.to(device), k_raw.to(device), v_raw.to(device), weight.to(device), weight.to(device), cos.to(device),
        sin.to(device), 1e-6, slots.to(device), kpd, vpd, bt.to(device), ctx.to(device), SCALE, exact=True)
    torch.cuda.synchronize()
    assert not got[1].any()
    flat_k, flat_v = kpd.view(-1, 8, 128).cpu(), vpd.view(-1, 8, 128).cpu()
    assert_bits(flat_k[5 * 16 + 9], kp.view(-1, 8, 128)[5 * 16 + 9])   # padding row: untouched
    assert_bits(flat_v[5 * 16 + 9], vp.view(-1, 8, 128)[5 * 16 + 9])
    assert_bits(flat_v[4 * 16 + 3], v_raw[0].view(8, 128))              # real rows: appended
    assert_bits(flat_v[7 * 16 + 0], v_raw[2].view(8, 128))


def test_exact_decode_prologue_matches_norm_rope_append_then_attend(device):
    """The prologue form (raw q / k / v rows in): q / k RMSNorm + RoPE, the K/V append at the slots,
    then attention -- output and both pools bit-identical to the oracle chain."""
    w = workloads.decode_step(seed=0)
    gen = torch.Generator().manual_seed(7)
    batch = 8
    q_raw = torch.randn(batch, 16 * 128, generator=gen).bfloat16()
    k_raw = torch.randn(batch, 8 * 128, generator=gen).bfloat16()
    v_raw = torch.randn(batch, 8 * 128, generator=gen).bfloat16()
    q_w = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16()
    k_w = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16()
    pos = torch.tensor([c - 1 for c in w.context_lens])
    inv = 1.0 / (1000000.0 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    freqs = pos.float().unsqueeze(-1) * inv
    emb = torch.cat((freqs, freqs), -1)
    cos, sin = emb.cos().bfloat16(), emb.sin().bfloat16()
    kp, vp = w.pools[0, 0].clone(), w.pools[0, 1].clone()
    kpd, vpd = kp.to(device), vp.to(device)
    got = data_plane.paged_decode_attention_fused(
        q_raw.to(device), k_raw.to(device), v_raw.to(device), q_w.to(device), k_w.to(device), cos.to(device),
        sin.to(device), 1e-6, w.slot_mapping.to(device), kpd, vpd, w.block_tables.to(device),
        torch.tensor(w.context_lens, device=device), SCALE, exact=True)

    def norm_rope(x, weight, heads):
        y = torch_ref.rms_norm_exact(x.view(batch, heads, 128), weight, 1e-6)
        rot = torch.cat((-y[..., 64:], y[..., :64]), -1)
        return y * cos.unsqueeze(1) + rot * sin.unsqueeze(1)

    kp.view(-1, 8, 128)[w.slot_mapping] = norm_rope(k_raw, k_w, 8)
    vp.view(-1, 8, 128)[w.slot_mapping] = v_raw.view(batch, 8, 128)
    want = torch_ref.paged_decode_attention(norm_rope(q_raw, q_w, 16), kp, vp, w.block_tables,
                                            torch.tensor(w.context_lens), SCALE, exact=True)
    assert_bits(got, want)
    assert_bits(kpd, kp)
    assert_bits(vpd, vp)


def prefill_case(seed, starts, lens, kv_heads, group):
    gen = torch.Generator().manual_seed(seed)
    width = max(lens)
    batch = len(lens)
    totals = [s + n for s, n in zip(starts, lens)]
    num_blocks = 1 + sum(-(-t // 16) for t in totals) + 4
    tables = workloads.permuted_tables(totals, num_blocks, gen)
    kp = torch.randn(num_blocks, 16, kv_heads, 128, generator=gen).bfloat16()
    vp = torch.randn(num_blocks, 16, kv_heads, 128, generator=gen).bfloat16()
    q = torch.randn(batch, group * kv_heads, width, 128, generator=gen).bfloat16()
    k = torch.randn(batch, kv_heads, width, 128, generator=gen).bfloat16()
    v = torch.randn(batch, width, kv_heads, 128, generator=gen).bfloat16().transpose(1, 2)  # a v_proj view
    nb = max(-(-s // 16) for s in starts)
    hist = torch.zeros((batch, nb), dtype=torch.long)
    for b, s in enumerate(starts):
        h = -(-s // 16)
        hist[b, :h] = torch.tensor(tables[b][:h], dtype=torch.long)
    return q, k, v, kp, vp, hist


@pytest.mark.parametrize("seed,starts,lens,group,kv_heads", [
    (0, [0], [37], 2, 8),
    (1, [0, 0], [64, 130], 2, 8),          # tile edges, left padding
    (2, [100, 2048], [300, 128], 2, 8),     # history of unequal lengths
    (3, [0, 33], [600, 517], 2, 8),
    (4, [1500], [400], 2, 8),
    (5, [30, 0], [100, 77], 5, 8),
    (6, [200], [90], 8, 2),
    (7, [70], [33], 1, 4),
    (9, [40, 0], [300, 45], 4, 8),          # Qwen3-4B / 8B's group: 4 query positions per workgroup
    (8, [5000], [700], 2, 8),               # 5.7k keys: past the LDS score cache, recomputed per pass
])
def test_exact_prefill_is_bit_identical_to_the_oracle(device, seed, starts, lens, group, kv_heads):
    """Real query rows bit-identical to the oracle (on the CPU and on cuda:0); left-padding rows
    zero (the reference attends them to the history, but nothing ever reads them)."""
    q, k, v, kp, vp, hist = prefill_case(seed, starts, lens, kv_heads, group)
    args = [t.to(device) for t in (q, k, v, kp, vp, hist)]
    got = data_plane.chunked_prefill_attention(*args, torch.tensor(starts, device=device),
                                               torch.tensor(lens, device=device), SCALE, exact=True).cpu()
    want_gpu = torch_ref.chunked_prefill_attention(args[0], args[1], args[2], (args[3], args[4]), args[5], starts,
                                                   lens, SCALE, exact=True).cpu()
    want_cpu = torch_ref.chunked_prefill_attention(q, k, v, (kp, vp), hist, starts, lens, SCALE, exact=True)
    ref = torch_ref.chunked_prefill_attention(q, k, v, (kp, vp), hist, starts, lens, SCALE)
    width = q.shape[2]
    for b, n in enumerate(lens):
        real = slice(width - n, width)
        assert_bits(got[b, real], want_gpu[b, real])
        assert_bits(got[b, real], want_cpu[b, real])
        assert (got[b, real].float() - ref[b, real].float()).abs().max().item() <= NEAR
        assert not got[b, :width - n].any()


def test_exact_prefill_query_load_forms_are_bit_identical(device):
    """Aligned query rows take 16-byte loads, others 2-byte loads: the same bits."""
    starts, lens = [60, 0], [150, 97]
    q, k, v, kp, vp, hist = prefill_case(11, starts, lens, 8, 2)
    args = [t.to(device) for t in (q, k, v, kp, vp, hist)]
    B, H, L, D = q.shape
    odd = torch.empty((B, H, L, D + 1), dtype=q.dtype, device=device)
    q_odd = odd[..., 1:]                                   # 2-byte offset, token stride D + 1
    q_odd.copy_(args[0])
    st, ln = torch.tensor(starts, device=device), torch.tensor(lens, device=device)
    aligned = data_plane.chunked_prefill_attention(*args, st, ln, SCALE, exact=True)
    unaligned = data_plane.chunked_prefill_attention(q_odd, *args[1:], st, ln, SCALE, exact=True)
    assert_bits(unaligned.cpu(), aligned.cpu())


def test_exact_rms_norm_is_bit_identical_to_the_oracle(device):
    gen = torch.Generator().manual_seed(0)
    x = (torch.randn(3000, 1024, generator=gen) * 3).bfloat16()
    r = torch.randn(3000, 1024, generator=gen).bfloat16()
    w = (1 + 0.1 * torch.randn(1024, generator=gen)).bfloat16()
    got, _ = data_plane.rms_norm(x.to(device), w.to(device), 1e-6)
    assert_bits(got, torch_ref.rms_norm_exact(x, w, 1e-6))
    got, h = data_plane.rms_norm(x.to(device), w.to(device), 1e-6, r.to(device))
    assert_bits(h, x + r)
    assert_bits(got, torch_ref.rms_norm_exact(x + r, w, 1e-6))
    # the op-for-op chain (ATen's fp32 sum) rounds the same way on almost every element
    xf = (x + r).float()
    chain = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    assert (got.cpu() != chain).float().mean().item() < 1e-4
