"""The oracle's exact-sum definitions (torch_ref.exact_sum, attend_exact, rms_norm_exact; the
numerics of the HIP model) pinned without the HIP code: exact sums against math.fsum, special cases
that fix the result, the fp64 textbook attention, agreement with the op-for-op restatement of the
reference (ATen's fp32 sums) to a bf16 ulp or two, independence from the summation order, and the
reference's own greedy tokens on the golden fixture (written by running the reference)."""

import json
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

from mini_infra_qwen3_amd.core import KVCacheManager
from mini_infra_qwen3_amd.model import Qwen3Config, Qwen3ForCausalLM
from oracle import closed_form, qwen3_ref, torch_ref

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import recipe  # noqa: E402

SCALE = 128 ** -0.5


# --------------------------------------------------------------------------- exact_sum
def test_exact_sum_is_the_correctly_rounded_sum_in_any_order():
    gen = torch.Generator().manual_seed(0)
    for trial in range(20):
        n = int(torch.randint(1, 5000, (1,), generator=gen))
        # fp32 values in [0, 1] spread over ~60 binades, as exp(s - m) gives them
        x = torch.exp(-torch.rand(n, generator=gen, dtype=torch.float64) * 40).float()
        x[0] = 1.0
        want = math.fsum(x.double().tolist())
        assert torch_ref.exact_sum(x).item() == want
        perm = x[torch.randperm(n, generator=gen)]
        assert torch_ref.exact_sum(perm).item() == want


def test_exact_sum_keeps_terms_a_plain_fp64_sum_loses():
    """1 followed by a thousand 2^-54: each addend is below half an ulp of the running sum."""
    x = torch.tensor([1.0] + [2.0 ** -54] * 1000, dtype=torch.float32)
    plain = sum(x.double().tolist())
    assert plain == 1.0
    assert torch_ref.exact_sum(x).item() == math.fsum(x.double().tolist()) == 1.0 + 1000 * 2.0 ** -54


# --------------------------------------------------------------------------- attention
def dense_case(seed, q_len, kv_len, heads=4, kv_heads=2, scale_q=1.0):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(1, heads, q_len, 128, generator=gen) * scale_q).bfloat16()
    k = torch.randn(1, kv_heads, kv_len, 128, generator=gen).bfloat16()
    v = torch.randn(1, kv_heads, kv_len, 128, generator=gen).bfloat16()
    return q, k, v


def bias_of(allowed):
    bias = torch.zeros(allowed.shape, dtype=torch.bfloat16)
    return bias.masked_fill(~allowed, torch.finfo(torch.bfloat16).min)


def test_one_visible_key_returns_its_value():
    q, k, v = dense_case(1, 3, 9)
    allowed = torch.zeros(1, 1, 3, 9, dtype=torch.bool)
    allowed[..., 0, 4] = allowed[..., 1, 0] = allowed[..., 2, 8] = True
    out = torch_ref.attend_exact(q, k, v, bias_of(allowed), SCALE).view(3, 4, 128)
    for i, t in enumerate((4, 0, 8)):
        for h in range(4):
            assert torch.equal(out[i, h], v[0, h // 2, t])


def test_equal_scores_average_the_values_with_rounded_weights():
    """Zero keys give every visible key score 0, so p = bf16(1 / n) and out = bf16(p * sum v)."""
    _, _, v = dense_case(2, 1, 37, heads=2, kv_heads=1)
    q = torch.ones(1, 2, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 1, 37, 128, dtype=torch.bfloat16)
    allowed = torch.ones(1, 1, 1, 37, dtype=torch.bool)
    allowed[..., 30:] = False
    out = torch_ref.attend_exact(q, k, v, bias_of(allowed), SCALE).view(2, 128)
    p = float(torch.tensor(1.0 / 30, dtype=torch.float32).bfloat16())
    sums = [math.fsum(p * float(x) for x in v[0, 0, :30, d].tolist()) for d in range(128)]
    want = torch.tensor(sums, dtype=torch.float64).float().bfloat16()
    assert torch.equal(out[0], want) and torch.equal(out[1], want)


def test_rows_with_nothing_visible_are_zero():
    q, k, v = dense_case(3, 2, 5)
    allowed = torch.ones(1, 1, 2, 5, dtype=torch.bool)
    allowed[..., 0, :] = False
    out = torch_ref.attend_exact(q, k, v, bias_of(allowed), SCALE)
    assert not out[0, 0].any() and out[0, 1].any()


@pytest.mark.parametrize("q_len,kv_len,scale_q", [(1, 500, 1.0), (7, 64, 0.5), (33, 300, 0.2)])
def test_attend_exact_matches_fp64_textbook(q_len, kv_len, scale_q):
    """Head mapping h // G, masking, the scale and the softmax against explicit fp64 loops (the
    bf16 rounding points leave a few ulps of |out| < 1)."""
    q, k, v = dense_case(4, q_len, kv_len, scale_q=scale_q)
    gen = torch.Generator().manual_seed(5)
    allowed = torch.rand(1, 1, q_len, kv_len, generator=gen) < 0.7
    allowed[..., 0] = True
    out = torch_ref.attend_exact(q, k, v, bias_of(allowed), SCALE).view(q_len, 4, 128).transpose(0, 1)
    ref = closed_form.prefill_attention_fp64(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(),
                                            allowed[0, 0].numpy(), SCALE)
    assert np.abs(out.float().numpy() - ref).max() < 1e-2


def test_attend_exact_is_within_rounding_of_the_op_for_op_restatement():
    """Same rounding points, different sums: at most a bf16 ulp or two apart, mostly identical."""
    q, k, v = dense_case(6, 16, 1000)
    allowed = torch.ones(1, 1, 16, 1000, dtype=torch.bool).tril(diagonal=984)
    exact = torch_ref.attend_exact(q, k, v, bias_of(allowed), SCALE)
    plain = torch_ref.attend(q, k, v, bias_of(allowed), SCALE)
    assert (exact.float() - plain.float()).abs().max().item() <= 4e-3
    assert (exact != plain).float().mean().item() < 0.02


def test_attend_exact_does_not_depend_on_the_key_order():
    """Scores spread over a wide range (many binades of exp) and 4096 keys, permuted."""
    q, k, v = dense_case(7, 4, 4096, scale_q=4.0)
    allowed = torch.ones(1, 1, 4, 4096, dtype=torch.bool)
    base = torch_ref.attend_exact(q, k, v, bias_of(allowed), SCALE)
    gen = torch.Generator().manual_seed(8)
    for _ in range(3):
        perm = torch.randperm(4096, generator=gen)
        assert torch.equal(torch_ref.attend_exact(q, k[:, :, perm], v[:, :, perm], bias_of(allowed), SCALE), base)


def test_paged_decode_exact_equals_dense_per_request():
    """Reference invariant (tests/unit/test_paged_kv_cache.py:109-163), bit for bit here."""
    gen = torch.Generator().manual_seed(9)
    ctx = [37, 5, 64]
    kp = torch.randn(32, 16, 2, 128, generator=gen).bfloat16()
    vp = torch.randn(32, 16, 2, 128, generator=gen).bfloat16()
    q = torch.randn(3, 4, 128, generator=gen).bfloat16()
    tables = torch.tensor([[3, 9, 1, 0], [12, 0, 0, 0], [7, 30, 2, 4]])
    got = torch_ref.paged_decode_attention(q, kp, vp, tables, torch.tensor(ctx), SCALE, exact=True).view(3, 4, 128)
    for b, n in enumerate(ctx):
        keys = torch.cat([kp[t] for t in tables[b]])[:n].transpose(0, 1).unsqueeze(0)
        vals = torch.cat([vp[t] for t in tables[b]])[:n].transpose(0, 1).unsqueeze(0)
        dense = torch_ref.attend_exact(q[b].view(1, 4, 1, 128), keys, vals, torch.zeros(1, 1, 1, n,
                                       dtype=torch.bfloat16), SCALE)
        assert torch.equal(got[b].reshape(-1), dense.reshape(-1))


# --------------------------------------------------------------------------- RMSNorm
def test_rms_norm_exact_of_a_constant_row_is_one():
    w = torch.ones(1024, dtype=torch.bfloat16)
    for c in (0.5, 2.0, -3.0, 17.0):
        x = torch.full((1, 1024), c, dtype=torch.bfloat16)
        out = torch_ref.rms_norm_exact(x, w, 1e-6)
        assert torch.equal(out, torch.full_like(out, math.copysign(1.0, c)))


def test_rms_norm_exact_is_within_an_ulp_of_the_aten_chain_and_order_free():
    gen = torch.Generator().manual_seed(10)
    x = (torch.randn(2000, 1024, generator=gen) * 3).bfloat16()
    w = (1 + 0.1 * torch.randn(1024, generator=gen)).bfloat16()
    exact = torch_ref.rms_norm_exact(x, w, 1e-6)
    xf = x.float()
    chain = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    diff = (exact.float() - chain.float()).abs()
    assert (diff <= chain.float().abs() * 2.0 ** -7).all()
    assert (exact != chain).float().mean().item() < 1e-3
    perm = torch.randperm(1024, generator=gen)
    assert torch.equal(torch_ref.rms_norm_exact(x[:, perm], w[perm], 1e-6), exact[:, perm])


# --------------------------------------------------------------------------- golden fixture
@pytest.fixture(scope="module")
def golden_model():
    cfg = Qwen3Config(**recipe.CONFIG, tie_word_embeddings=False)
    shapes = {n: tuple(p.shape) for n, p in Qwen3ForCausalLM(cfg).state_dict().items()}
    meta = json.loads((GOLDEN / "reference_bf16.json").read_text())
    return qwen3_ref.ReferenceQwen3(cfg, recipe.state_dict(shapes), exact=True), meta


def test_exact_attention_is_within_an_ulp_of_the_reference_run():
    tensors = load_file(str(GOLDEN / "reference_bf16.safetensors"))
    for name, inputs in (("attend_decode_out", recipe.attend_decode_inputs()),
                         ("attend_prefill_out", recipe.attend_prefill_inputs())):
        want = tensors[name].float()
        got = torch_ref.attend_exact(*inputs, SCALE).float()
        assert ((got - want).abs() <= want.abs() * 2.0 ** -7 + 1e-6).all(), name


def test_exact_model_gives_the_reference_runs_greedy_tokens(golden_model):
    """Whole-prompt prefill, paged decode steps and chunked prefill with history: the tokens the
    reference produced (tests/golden/make_golden.py)."""
    model, meta = golden_model
    prompts = recipe.prompts(recipe.PREFILL_PROMPT_LENS, "prefill_prompts")
    manager = KVCacheManager(recipe.BLOCK_SIZE, 24)
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(len(prompts))]
    pools = torch_ref.make_pools(2, 24, recipe.BLOCK_SIZE, 8, 128)
    tokens, presents = qwen3_ref.prefill(model, prompts)
    assert tokens == meta["prefill_tokens"]
    qwen3_ref.store_prefill(pools, presents, tables, [len(p) for p in prompts], [0] * 3, recipe.BLOCK_SIZE)
    lengths = [len(p) for p in prompts]
    for step in range(recipe.DECODE_STEPS):
        for i in range(3):
            manager.allocate_slots(i, 1)
        tables = [manager.block_table(i) for i in range(3)]
        tokens = qwen3_ref.decode_step(model, tables, tokens, lengths, pools, recipe.BLOCK_SIZE).argmax(-1).tolist()
        assert tokens == meta["decode_tokens"][step]
        lengths = [n + 1 for n in lengths]
    prompts = recipe.prompts(recipe.CHUNK_PROMPT_LENS, "chunk_prompts")
    pools = torch_ref.make_pools(2, 16, recipe.BLOCK_SIZE, 8, 128)
    for k, (starts, ends) in enumerate((([0, 0], recipe.CHUNK_CUTS),
                                        (recipe.CHUNK_CUTS, [len(p) for p in prompts]))):
        chunks = [p[s:e] for p, s, e in zip(prompts, starts, ends)]
        toks, presents = qwen3_ref.prefill_chunk_step(model, chunks, starts, meta["chunk_tables"], pools,
                                                      recipe.BLOCK_SIZE)
        qwen3_ref.store_prefill(pools, presents, meta["chunk_tables"], [e - s for s, e in zip(starts, ends)], starts,
                                recipe.BLOCK_SIZE)
        assert toks == meta["chunk_tokens"][k]
