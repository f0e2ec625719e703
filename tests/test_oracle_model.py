"""Pins the oracle's Qwen3 / PagedRunner restatement with the invariants of the reference suite
(tests/unit/test_paged_kv_cache.py:109-262), run in fp32 on the CPU on a tiny model like the
reference's own fixture (build_tiny_model + untied head: tests/unit/conftest.py:13-25)."""

from dataclasses import dataclass

import pytest
import torch

from oracle import qwen3_ref, torch_ref


@dataclass
class TinyConfig:
    vocab_size: int = 97
    hidden_size: int = 32
    intermediate_size: int = 64
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 4
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0


def tiny_model(seed=0, head_seed=1234) -> qwen3_ref.ReferenceQwen3:
    c = TinyConfig()
    gen = torch.Generator().manual_seed(seed)
    sd = {"model.embed_tokens.weight": torch.randn(c.vocab_size, c.hidden_size, generator=gen) * 0.5,
          "model.norm.weight": torch.ones(c.hidden_size)}
    for i in range(c.num_hidden_layers):
        p = f"model.layers.{i}."
        qd, kd = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
        for name, shape in (("self_attn.q_proj", (qd, c.hidden_size)), ("self_attn.k_proj", (kd, c.hidden_size)),
                            ("self_attn.v_proj", (kd, c.hidden_size)), ("self_attn.o_proj", (c.hidden_size, qd)),
                            ("mlp.gate_proj", (c.intermediate_size, c.hidden_size)),
                            ("mlp.up_proj", (c.intermediate_size, c.hidden_size)),
                            ("mlp.down_proj", (c.hidden_size, c.intermediate_size))):
            sd[p + name + ".weight"] = torch.randn(shape, generator=gen) * 0.3
        for name, n in (("self_attn.q_norm", c.head_dim), ("self_attn.k_norm", c.head_dim),
                        ("input_layernorm", c.hidden_size), ("post_attention_layernorm", c.hidden_size)):
            sd[p + name + ".weight"] = torch.ones(n)
    sd["lm_head.weight"] = torch.randn(c.vocab_size, c.hidden_size, generator=torch.Generator().manual_seed(head_seed))
    return qwen3_ref.ReferenceQwen3(c, sd)


def pools_for(model, num_blocks, block_size):
    c = model.config
    return torch_ref.make_pools(c.num_hidden_layers, num_blocks, block_size, c.num_key_value_heads, c.head_dim,
                                dtype=torch.float32)


def tables_from(num_tokens, block_size, first_block):
    nb = -(-num_tokens // block_size)
    return list(range(first_block, first_block + nb))


@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_paged_decode_equals_dense_decode(block_size):
    """tests/unit/test_paged_kv_cache.py:109-163 on the oracle: logits within 1e-4, same tokens."""
    model = tiny_model()
    prompts = [[3, 5, 7, 9, 11, 13, 15], [17, 19, 23], [29]]
    steps = 5
    pools = pools_for(model, 64, block_size)
    tables, nxt = [], 1
    for p in prompts:
        tables.append(tables_from(len(p) + steps, block_size, nxt))
        nxt += len(tables[-1])
    _, presents = qwen3_ref.prefill(model, prompts)
    qwen3_ref.store_prefill(pools, presents, tables, [len(p) for p in prompts], [0] * 3, block_size)
    dense = [qwen3_ref.prefill(model, [p])[1] for p in prompts]
    tokens = [[(i * 13 + 2) % 90 + 1] for i in range(3)]
    lengths = [len(p) for p in prompts]
    for _ in range(steps):
        paged = qwen3_ref.decode_step(model, tables, [t[-1] for t in tokens], lengths, pools, block_size)
        for i in range(3):
            logits, dense[i] = model.forward(torch.tensor([[tokens[i][-1]]]), position_ids=torch.tensor([[lengths[i]]]),
                                             past_key_values=dense[i])
            assert (paged[i] - logits[0, -1]).abs().max().item() <= 1e-4
            assert int(paged[i].argmax()) == int(logits[0, -1].argmax())
            lengths[i] += 1
            tokens[i].append(int(paged[i].argmax()))


@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_chunked_prefill_equals_one_shot(block_size):
    """tests/unit/test_paged_kv_cache.py:210-246 on the oracle: pool K/V and first tokens."""
    model = tiny_model()
    prompts = [[(j * 5 + 3) % 80 + 1 for j in range(11)], [(j * 7 + 2) % 80 + 1 for j in range(6)]]
    rounds = [[(0, 0, 5), (1, 0, 2)], [(0, 5, 8), (1, 2, 6)], [(0, 8, 11)]]
    pools = pools_for(model, 64, block_size)
    tables = [tables_from(11, block_size, 1), tables_from(6, block_size, 1 + len(tables_from(11, block_size, 1)))]
    first = {}
    for chunks in rounds:
        bt = [tables[r] for r, _, _ in chunks]
        starts = [s for _, s, _ in chunks]
        toks, presents = qwen3_ref.prefill_chunk_step(model, [prompts[r][s:e] for r, s, e in chunks], starts, bt,
                                                      pools, block_size)
        qwen3_ref.store_prefill(pools, presents, bt, [e - s for _, s, e in chunks], starts, block_size)
        for (r, _, e), t in zip(chunks, toks):
            if e == len(prompts[r]):
                first[r] = t
    for r, p in enumerate(prompts):
        toks, ref = qwen3_ref.prefill(model, [p])
        assert first[r] == toks[0]
        for layer, (k, v) in enumerate(ref):
            kp, vp = pools[layer]
            got_k = torch.cat([kp[b] for b in tables[r]])[:len(p)].transpose(0, 1)
            got_v = torch.cat([vp[b] for b in tables[r]])[:len(p)].transpose(0, 1)
            torch.testing.assert_close(got_k, k[0], atol=1e-5, rtol=0)
            torch.testing.assert_close(got_v, v[0], atol=1e-5, rtol=0)


def test_chunk_without_history_is_whole_prompt_prefill():
    """tests/unit/test_paged_kv_cache.py:249-262 on the oracle: bitwise identical."""
    model = tiny_model()
    prompts = [[3, 5, 7, 9, 11, 13], [17, 19, 23]]
    pools = pools_for(model, 16, 4)
    toks_c, cache_c = qwen3_ref.prefill_chunk_step(model, prompts, [0, 0], [[1, 2], [3]], pools, 4)
    toks_w, cache_w = qwen3_ref.prefill(model, prompts)
    assert toks_c == toks_w
    for (kc, vc), (kw, vw) in zip(cache_c, cache_w):
        assert torch.equal(kc, kw) and torch.equal(vc, vw)



def serial_generate(model, prompt, max_new):
    """One request alone: whole-prompt prefill, then dense-cache decode (reference serial baseline,
    tests/unit/test_paged_scheduler.py:30-45)."""
    toks, cache = qwen3_ref.prefill(model, [prompt])
    out = [toks[0]]
    for k in range(max_new - 1):
        logits, cache = model.forward(torch.tensor([[out[-1]]]), position_ids=torch.tensor([[len(prompt) + k]]),
                                      past_key_values=cache)
        out.append(int(logits[0, -1].argmax()))
    return out


@pytest.mark.parametrize("budget,capacity,block_size", [(8, 2, 4), (5, 3, 1), (64, 4, 16)])
def test_scheduled_paged_run_matches_serial_generation(budget, capacity, block_size):
    """tests/unit/test_paged_scheduler.py:368-390 on the oracle backend: continuous batching with
    chunked prefill produces each request's serial greedy sequence."""
    from mini_infra_qwen3_amd.core import Request
    from mini_infra_qwen3_amd.engine import run_scheduler

    model = tiny_model()
    prompts = [[(j * 7 + i * 3) % 90 + 1 for j in range(n)] for i, n in enumerate([13, 4, 9, 2, 16])]
    budgets = [5, 7, 3, 6, 4]
    requests = [Request(i, tuple(p), m, a) for i, (p, m, a) in enumerate(zip(prompts, budgets, [0, 0, 0, 1, 2]))]
    backend = qwen3_ref.ReferenceScheduleBackend(model, requests, capacity, block_size=block_size)
    result = run_scheduler(backend, requests, token_budget=budget, max_running_requests=capacity,
                           step_clock=lambda out: 1.0)
    for i, (p, m) in enumerate(zip(prompts, budgets)):
        assert result.tokens[i] == serial_generate(model, p, m)


@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_mixed_step_equals_chunk_step_plus_decode_step(block_size):
    """The oracle's mixed step (prompt chunks and decode tokens in one flattened forward; the
    reference defines no such step) against the reference's own two steps on the same state: a
    chunk step over the same chunks (``prefill_chunk_logits``) and a decode step over the same
    tokens (``decode_step``).  fp32 on the CPU: logits within rounding, the same greedy tokens, the
    same chunk K/V and the same pools after the decode append."""
    model = tiny_model(seed=3)
    gen = torch.Generator().manual_seed(block_size)
    prompt_a = torch.randint(1, 97, (10,), generator=gen).tolist()   # prefilled; decodes one token
    prompt_b = torch.randint(1, 97, (13,), generator=gen).tolist()   # first 7 prefilled; chunk 7..12
    prompt_c = torch.randint(1, 97, (5,), generator=gen).tolist()    # a fresh chunk
    table_a = tables_from(11, block_size, 1)
    table_b = tables_from(13, block_size, 1 + len(table_a))
    table_c = tables_from(5, block_size, 1 + len(table_a) + len(table_b))
    pools = pools_for(model, 1 + len(table_a) + len(table_b) + len(table_c), block_size)
    _, presents = qwen3_ref.prefill_chunk_logits(model, [prompt_a, prompt_b[:7]], [0, 0], [table_a, table_b], pools,
                                                 block_size)
    qwen3_ref.store_prefill(pools, presents, [table_a, table_b], [10, 7], [0, 0], block_size)
    last_a = int(torch.randint(1, 97, (1,), generator=gen))

    two = [(k.clone(), v.clone()) for k, v in pools]
    chunk_logits, chunk_presents = qwen3_ref.prefill_chunk_logits(model, [prompt_b[7:], prompt_c], [7, 0],
                                                                  [table_b, table_c], two, block_size)
    decode_logits = qwen3_ref.decode_step(model, [table_a], [last_a], [10], two, block_size)

    one = [(k.clone(), v.clone()) for k, v in pools]
    mixed_logits, mixed_presents = qwen3_ref.mixed_step_logits(model, [prompt_b[7:], prompt_c], [7, 0],
                                                               [table_b, table_c], [last_a], [10], [table_a], one,
                                                               block_size)
    want = torch.cat((chunk_logits, decode_logits))
    assert mixed_logits.shape == want.shape
    torch.testing.assert_close(mixed_logits, want, rtol=1e-5, atol=1e-5)
    assert mixed_logits.argmax(-1).tolist() == want.argmax(-1).tolist()
    width = 6
    for (mk, mv), (ck, cv) in zip(mixed_presents, chunk_presents):
        assert mk.shape[2] == width
        for row, n in enumerate((6, 5)):  # real tokens (the chunk step also caches its pad tokens' K/V)
            torch.testing.assert_close(mk[row, :, -n:], ck[row, :, -n:], rtol=1e-5, atol=1e-5)
            torch.testing.assert_close(mv[row, :, -n:], cv[row, :, -n:], rtol=1e-5, atol=1e-5)
    for (ok, ov), (tk, tv) in zip(one, two):
        torch.testing.assert_close(ok, tk, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(ov, tv, rtol=1e-5, atol=1e-5)


def test_padded_mixed_step_equals_the_unpadded_one():
    """The oracle's mixed step at a padded shape (pad chunk tokens after the ragged rows, pad decode
    rows: the shape a mixed step with reference numerics runs at) against the unpadded step on the
    same state: the same logits for the real rows (within fp32 rounding on the CPU: only the
    GEMMs' M differs), the same chunk K/V, pad decode rows writing nothing to the pools."""
    block_size = 4
    model = tiny_model(seed=5)
    gen = torch.Generator().manual_seed(11)
    prompt_a = torch.randint(1, 97, (10,), generator=gen).tolist()
    prompt_b = torch.randint(1, 97, (13,), generator=gen).tolist()
    prompt_c = torch.randint(1, 97, (5,), generator=gen).tolist()
    table_a = tables_from(11, block_size, 1)
    table_b = tables_from(13, block_size, 1 + len(table_a))
    table_c = tables_from(5, block_size, 1 + len(table_a) + len(table_b))
    pools = pools_for(model, 1 + len(table_a) + len(table_b) + len(table_c), block_size)
    _, presents = qwen3_ref.prefill_chunk_logits(model, [prompt_a, prompt_b[:7]], [0, 0], [table_a, table_b], pools,
                                                 block_size)
    qwen3_ref.store_prefill(pools, presents, [table_a, table_b], [10, 7], [0, 0], block_size)
    args = ([prompt_b[7:], prompt_c], [7, 0], [table_b, table_c], [int(prompt_a[-1])], [10], [table_a])
    plain_pools = [(k.clone(), v.clone()) for k, v in pools]
    padded_pools = [(k.clone(), v.clone()) for k, v in pools]
    plain, plain_kv = qwen3_ref.mixed_step_logits(model, *args, plain_pools, block_size)
    padded, padded_kv = qwen3_ref.mixed_step_logits(model, *args, padded_pools, block_size, chunk_tokens=16,
                                                    decode_rows=4)
    assert padded.shape == plain.shape == (3, model.config.vocab_size)
    torch.testing.assert_close(padded, plain, rtol=1e-5, atol=1e-5)
    assert padded.argmax(-1).tolist() == plain.argmax(-1).tolist()
    for (pk, pv), (k, v) in zip(padded_kv, plain_kv):
        assert pk.shape == k.shape and k.shape[2] == 6
        torch.testing.assert_close(pk, k, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(pv, v, rtol=1e-5, atol=1e-5)
    for (pk, pv), (k, v) in zip(padded_pools, plain_pools):
        torch.testing.assert_close(pk, k, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(pv, v, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError, match="below the step"):
        qwen3_ref.mixed_step_logits(model, *args, [(k.clone(), v.clone()) for k, v in pools], block_size,
                                    chunk_tokens=10)
