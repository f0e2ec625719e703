"""PagedRunner + Qwen3 on the GPU against the oracle's restatement of the reference runner and
model, same bf16 weights, in the scenarios of the reference suite (tests/unit/test_paged_kv_cache.py)
at the Qwen3 attention shape (16 / 8 heads of 128, block 16).

The model runs reference numerics (its default: the reference's rounding points with exact sums,
the reference's GEMM calls).  The oracle runs twice:
* with the same numerics on cuda:0 (``ReferenceQwen3(exact=True)``), where its GEMMs are the
  product's own: logits, greedy tokens and every stored K/V row must be bit-identical;
* op for op on the CPU (ATen's fp32 sums): greedy tokens must agree and logits / K/V stay within
  bf16 rounding (``LOGIT_RTOL``, ``DEEP_ATOL``: a wrong block, slot or position moves values by O(1)).
Graph tests with padded buckets run the model's bandwidth form (``exact=False``)."""

import pytest
import torch

from mini_infra_qwen3_amd.core import KVCacheManager
from mini_infra_qwen3_amd.model import Qwen3Config, Qwen3ForCausalLM, init_random_
from mini_infra_qwen3_amd.worker import PagedKVCachePool, PagedRunner
from oracle import qwen3_ref, torch_ref

pytestmark = pytest.mark.gpu

BS = 16
DEEP_ATOL = 5e-2  # K/V of layers after the first attention: a few bf16 ulps at |x| < 8
LOGIT_RTOL = 2e-2  # logits: fraction of the step's largest |logit|


def small_config(layers=2):
    return Qwen3Config(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                       num_attention_heads=16, num_key_value_heads=8, head_dim=128)


@pytest.fixture(scope="module")
def models():
    """(product model on cuda:0, oracle with the same numerics on cuda:0, op-for-op oracle on the
    CPU), identical bf16 weights, untied head."""
    cfg = small_config()
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, seed=0, std=0.05, untied_head_seed=1234)
    model = model.to(torch.bfloat16)
    weights = {k: v.clone() for k, v in model.state_dict().items()}
    return (model.to("cuda:0").eval(), qwen3_ref.ReferenceQwen3(cfg, weights, "cuda:0", exact=True),
            qwen3_ref.ReferenceQwen3(cfg, weights))


@pytest.fixture(scope="module")
def fast_model(models):
    """The same weights in the bandwidth form (fp32 online-softmax kernels, concatenated GEMMs)."""
    model = Qwen3ForCausalLM(small_config(), exact=False)
    init_random_(model, seed=0, std=0.05, untied_head_seed=1234)
    model = model.to(torch.bfloat16).to("cuda:0").eval()
    for (name, a), (_, b) in zip(model.state_dict().items(), models[0].state_dict().items()):
        assert torch.equal(a, b), name
    return model


def assert_bits(got, want):
    g, w = got.contiguous().view(torch.int16), want.contiguous().view(torch.int16)
    assert torch.equal(g, w), f"{(g != w).sum().item()} of {g.numel()} values differ"


def assert_kv_near(got, want):
    """Against the op-for-op oracle on the CPU: other GEMMs and fp32 sums, values within rounding."""
    assert (got.float().cpu() - want.float().cpu()).abs().max().item() <= DEEP_ATOL


def assert_kv_close(layer, got, want):
    got, want = got.float().cpu(), want.float().cpu()
    if layer == 0:
        assert ((got - want).abs() <= want.abs() * 2.0 ** -7).all()
    else:
        assert (got - want).abs().max().item() <= DEEP_ATOL


def make_pool(cfg, num_blocks, block_size=BS):
    return PagedKVCachePool(cfg.num_hidden_layers, num_blocks, block_size, cfg.num_key_value_heads, cfg.head_dim,
                            torch.bfloat16, "cuda:0")


def request_kv(pool, layer, table, length):
    key_pool, value_pool = pool.kv_pools[layer]
    k = torch.cat([key_pool[b] for b in table])[:length].transpose(0, 1)
    v = torch.cat([value_pool[b] for b in table])[:length].transpose(0, 1)
    return k, v


def prompts_of(lengths, seed=0):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randint(1, 999, (n,), generator=gen).tolist() for n in lengths]


def test_pool_layout_and_byte_accounting(models):
    model = models[0]
    cfg = model.config
    pool = make_pool(cfg, 10)
    key_pool, value_pool = pool.kv_pools[0]
    assert len(pool.kv_pools) == cfg.num_hidden_layers
    assert tuple(key_pool.shape) == (10, BS, 8, 128) == tuple(value_pool.shape)
    assert not key_pool.any() and not value_pool.any()
    assert pool.bytes_per_block == 2 * cfg.num_hidden_layers * BS * 8 * 128 * 2
    assert pool.total_bytes == 10 * pool.bytes_per_block


def test_prepare_decode_inputs_packs_reference_metadata(models):
    model = models[0]
    runner = PagedRunner(model)
    ids, pos, meta = runner.prepare_decode_inputs([[9, 4], [7]], last_tokens=[11, 22], positions=[21, 2],
                                                  block_size=BS)
    assert ids.tolist() == [[11], [22]] and pos.tolist() == [[21], [2]]
    assert meta.slot_mapping.tolist() == [4 * BS + 5, 7 * BS + 2]
    assert meta.context_lens.tolist() == [22, 3]
    assert meta.block_tables.tolist() == [[9, 4], [7, 0]]


def test_store_prefill_matches_oracle_and_isolates_requests(models):
    """Left-padded batched prefill scattered to each request's blocks (test_paged_kv_cache.py:67-93)."""
    model, ref, ref_cpu = models
    prompts = prompts_of([37, 20], seed=1)
    manager = KVCacheManager(BS, num_blocks=16)
    manager.allocate_slots(5, 40)  # someone else's blocks first: tables are not 1, 2, ...
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    pool = make_pool(model.config, 16)
    runner = PagedRunner(model)
    out = runner.run_prefill_step(prompts)
    runner.store_prefill(pool, out.prefill_cache, [manager.block_table(i) for i in range(2)], [37, 20], [0, 0])
    first, presents = qwen3_ref.prefill(ref, prompts)
    cpu_first, cpu_presents = qwen3_ref.prefill(ref_cpu, prompts)
    assert out.next_tokens == first == cpu_first
    for i, p in enumerate(prompts):
        width = presents[0][0].shape[2]
        for layer in range(model.config.num_hidden_layers):
            k, v = request_kv(pool, layer, manager.block_table(i), len(p))
            assert_bits(k, presents[layer][0][i, :, width - len(p):])
            assert_bits(v, presents[layer][1][i, :, width - len(p):])
            assert_kv_near(k, cpu_presents[layer][0][i, :, width - len(p):])
            assert_kv_near(v, cpu_presents[layer][1][i, :, width - len(p):])
    for b in manager.block_table(5):
        assert not pool.kv_pools[0][0][b].any()


@pytest.mark.parametrize("bs", [BS, 2 * BS], ids=["block16", "block32"])
def test_paged_decode_matches_oracle_tokens_and_logits(models, bs):
    """Mixed-length requests decoded step by step (test_paged_kv_cache.py:109-163): logits and every
    K/V row bit-identical to the oracle with the same numerics, greedy tokens identical to it and to
    the op-for-op oracle on the CPU, logits within rounding of the latter.  A 32-token block pool
    runs the kernels on 16-token sub-blocks."""
    model, ref, ref_cpu = models
    cfg = model.config
    prompts = prompts_of([45, 17, 3], seed=2)
    steps = 6
    manager = KVCacheManager(bs, num_blocks=64)
    pool = make_pool(cfg, 64, bs)
    ref_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, bs, 8, 128, device="cuda:0")
    cpu_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, bs, 8, 128)
    runner = PagedRunner(model)
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(3)]
    out = runner.run_prefill_step(prompts)
    runner.store_prefill(pool, out.prefill_cache, tables, [len(p) for p in prompts], [0] * 3)
    first, presents = qwen3_ref.prefill(ref, prompts)
    qwen3_ref.store_prefill(ref_pools, presents, tables, [len(p) for p in prompts], [0] * 3, bs)
    _, cpu_presents = qwen3_ref.prefill(ref_cpu, prompts)
    qwen3_ref.store_prefill(cpu_pools, cpu_presents, tables, [len(p) for p in prompts], [0] * 3, bs)
    assert out.next_tokens == first
    tokens = [[t] for t in first]
    lengths = [len(p) for p in prompts]
    with torch.inference_mode():
        for _ in range(steps):
            for i in range(3):
                assert manager.allocate_slots(i, 1)
            tables = [manager.block_table(i) for i in range(3)]
            ids, pos, meta = runner.prepare_decode_inputs(tables, [t[-1] for t in tokens], lengths, bs)
            logits = model(ids, position_ids=pos, attn_metadata=meta._replace(kv_pools=tuple(pool.kv_pools)),
                           last_logits_only=True)[0][:, -1].float()
            got = runner.run_decode_step(ids, pos, meta, pool)  # rewrites the same rows: same inputs
            want = qwen3_ref.decode_step(ref, tables, [t[-1] for t in tokens], lengths, ref_pools, bs).float()
            want_cpu = qwen3_ref.decode_step(ref_cpu, tables, [t[-1] for t in tokens], lengths, cpu_pools, bs)
            assert torch.equal(logits, want)
            assert got.next_tokens == logits.argmax(-1).tolist() == want.argmax(-1).tolist()
            assert got.next_tokens == want_cpu.argmax(-1).tolist()
            assert (logits.cpu() - want_cpu.float()).abs().max().item() <= LOGIT_RTOL * want_cpu.float().abs().max().item()
            for i in range(3):
                lengths[i] += 1
                tokens[i].append(got.next_tokens[i])
    for i in range(3):  # prefill- and decode-written K/V rows: the oracle's, bit for bit
        for layer in range(cfg.num_hidden_layers):
            for kv in range(2):
                got = request_kv(pool, layer, manager.block_table(i), lengths[i])[kv]
                want = torch.cat([ref_pools[layer][kv][b] for b in manager.block_table(i)])[:lengths[i]]
                assert_bits(got, want.transpose(0, 1))
                want = torch.cat([cpu_pools[layer][kv][b] for b in manager.block_table(i)])[:lengths[i]]
                assert_kv_near(got, want.transpose(0, 1))


@pytest.mark.parametrize("heads,kv_heads", [(16, 4), (20, 4), (32, 4), (8, 8)], ids=["gqa4", "gqa5", "gqa8", "mha"])
def test_other_gqa_groups_decode_like_the_oracle(heads, kv_heads):
    """Models whose query heads share KV heads in groups other than 2 (Qwen3-4B/8B: 4, Qwen3-14B:
    5, Qwen3-32B: 8; multi-head: 1): prefill, then decode steps through the fused decode kernel,
    give the oracle's logits bit for bit and so its greedy tokens."""
    cfg = Qwen3Config(vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=128)
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, seed=3, std=0.05, untied_head_seed=99)
    model = model.to(torch.bfloat16)
    ref = qwen3_ref.ReferenceQwen3(cfg, {k: v.clone() for k, v in model.state_dict().items()}, "cuda:0", exact=True)
    model = model.to("cuda:0").eval()
    prompts = prompts_of([45, 17, 3], seed=4)
    manager = KVCacheManager(BS, num_blocks=32)
    pool = make_pool(cfg, 32)
    ref_pools = torch_ref.make_pools(cfg.num_hidden_layers, 32, BS, kv_heads, 128, device="cuda:0")
    runner = PagedRunner(model)
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(3)]
    lengths = [len(p) for p in prompts]
    out = runner.run_prefill_step(prompts)
    runner.store_prefill(pool, out.prefill_cache, tables, lengths, [0] * 3)
    first, presents = qwen3_ref.prefill(ref, prompts)
    qwen3_ref.store_prefill(ref_pools, presents, tables, lengths, [0] * 3, BS)
    assert out.next_tokens == first
    last = list(first)
    with torch.inference_mode():
        for _ in range(4):
            for i in range(3):
                assert manager.allocate_slots(i, 1)
            tables = [manager.block_table(i) for i in range(3)]
            ids, pos, meta = runner.prepare_decode_inputs(tables, last, lengths, BS)
            logits = model(ids, position_ids=pos, attn_metadata=meta._replace(kv_pools=tuple(pool.kv_pools)),
                           last_logits_only=True)[0][:, -1].float()
            got = runner.run_decode_step(ids, pos, meta, pool)
            want = qwen3_ref.decode_step(ref, tables, last, lengths, ref_pools, BS).float()
            assert torch.equal(logits, want)
            assert got.next_tokens == logits.argmax(-1).tolist() == want.argmax(-1).tolist()
            lengths = [n + 1 for n in lengths]
            last = got.next_tokens


def test_stale_data_in_recycled_blocks_is_masked(models):
    """test_paged_kv_cache.py:166-207: a request reusing freed, unzeroed blocks decodes exactly as
    one on a fresh pool."""
    model = models[0]
    runner = PagedRunner(model)

    def decode_once(manager, pool, idx, prompt):
        manager.allocate_slots(idx, len(prompt))
        out = runner.run_prefill_step([prompt])
        runner.store_prefill(pool, out.prefill_cache, [manager.block_table(idx)], [len(prompt)], [0])
        manager.allocate_slots(idx, 1)
        ids, pos, meta = runner.prepare_decode_inputs([manager.block_table(idx)], [7], [len(prompt)], BS)
        with torch.inference_mode():
            logits, _ = model(ids, position_ids=pos, attn_metadata=meta._replace(kv_pools=tuple(pool.kv_pools)))
        return logits

    manager = KVCacheManager(BS, num_blocks=8)
    pool = make_pool(model.config, 8)
    decode_once(manager, pool, 0, prompts_of([40], seed=3)[0])  # fills blocks 1-3 with data
    manager.free(0)
    recycled = decode_once(manager, pool, 1, [17, 19, 23, 29, 31])
    fresh = decode_once(KVCacheManager(BS, num_blocks=8), make_pool(model.config, 8), 1, [17, 19, 23, 29, 31])
    assert torch.equal(recycled, fresh)


def test_chunked_prefill_matches_one_shot(models):
    """test_paged_kv_cache.py:210-246 at block 16: rows with different starts, history of unequal
    length; pool K/V close to the one-shot prefill, first tokens equal."""
    model = models[0]
    cfg = model.config
    prompts = prompts_of([75, 40], seed=4)
    rounds = [[(0, 0, 20), (1, 0, 9)], [(0, 20, 52), (1, 9, 33)], [(0, 52, 75), (1, 33, 40)]]
    manager = KVCacheManager(BS, num_blocks=64)
    pool = make_pool(cfg, 64)
    runner = PagedRunner(model)
    first = {}
    with torch.inference_mode():
        for chunks in rounds:
            for r, s, e in chunks:
                assert manager.allocate_slots(r, e - s)
            tables = [manager.block_table(r) for r, _, _ in chunks]
            starts = [s for _, s, _ in chunks]
            out = runner.run_prefill_chunk_step([prompts[r][s:e] for r, s, e in chunks], starts, tables, pool)
            runner.store_prefill(pool, out.prefill_cache, tables, [e - s for _, s, e in chunks], starts)
            for (r, _, e), t in zip(chunks, out.next_tokens):
                if e == len(prompts[r]):
                    first[r] = t
    for r, p in enumerate(prompts):
        whole = runner.run_prefill_step([p])
        assert first[r] == whole.next_tokens[0]
        for layer in range(cfg.num_hidden_layers):
            k, v = request_kv(pool, layer, manager.block_table(r), len(p))
            wk, wv = whole.prefill_cache[layer]  # other GEMM shapes: no bitwise claim even at layer 0
            assert (k.float() - wk[0].float()).abs().max().item() <= DEEP_ATOL
            assert (v.float() - wv[0].float()).abs().max().item() <= DEEP_ATOL


def test_chunk_without_history_is_bitwise_whole_prompt_prefill(models):
    """test_paged_kv_cache.py:249-262: start 0 everywhere runs the same path as a whole prefill."""
    model = models[0]
    prompts = prompts_of([30, 12], seed=5)
    runner = PagedRunner(model)
    pool = make_pool(model.config, 16)
    chunk = runner.run_prefill_chunk_step(prompts, [0, 0], [[1, 2], [3]], pool)
    whole = runner.run_prefill_step(prompts)
    assert chunk.next_tokens == whole.next_tokens
    for (kc, vc), (kw, vw) in zip(chunk.prefill_cache, whole.prefill_cache):
        assert torch.equal(kc, kw) and torch.equal(vc, vw)


def test_chunked_prefill_matches_oracle_runner(models):
    """One chunk step with history through both runners: same first tokens; stored K/V bit-identical
    to the oracle with the same numerics, close to the op-for-op oracle's."""
    model, ref, ref_cpu = models
    cfg = model.config
    prompts = prompts_of([50, 33], seed=6)
    manager = KVCacheManager(BS, num_blocks=32)
    pool = make_pool(cfg, 32)
    ref_pools = torch_ref.make_pools(cfg.num_hidden_layers, 32, BS, 8, 128, device="cuda:0")
    cpu_pools = torch_ref.make_pools(cfg.num_hidden_layers, 32, BS, 8, 128)
    runner = PagedRunner(model)
    for r, p in enumerate(prompts):
        manager.allocate_slots(r, len(p))
    tables = [manager.block_table(r) for r in range(2)]
    cut = [21, 16]
    for chunk_id in range(2):
        starts = [0, 0] if chunk_id == 0 else cut
        ends = cut if chunk_id == 0 else [len(p) for p in prompts]
        chunks = [p[s:e] for p, s, e in zip(prompts, starts, ends)]
        out = runner.run_prefill_chunk_step(chunks, starts, tables, pool)
        runner.store_prefill(pool, out.prefill_cache, tables, [e - s for s, e in zip(starts, ends)], starts)
        lens = [e - s for s, e in zip(starts, ends)]
        toks, presents = qwen3_ref.prefill_chunk_step(ref, chunks, starts, tables, ref_pools, BS)
        qwen3_ref.store_prefill(ref_pools, presents, tables, lens, starts, BS)
        toks_cpu, cpu_presents = qwen3_ref.prefill_chunk_step(ref_cpu, chunks, starts, tables, cpu_pools, BS)
        qwen3_ref.store_prefill(cpu_pools, cpu_presents, tables, lens, starts, BS)
        if chunk_id == 1:
            assert out.next_tokens == toks == toks_cpu
    for r, p in enumerate(prompts):
        for layer in range(cfg.num_hidden_layers):
            for kv in range(2):
                got = request_kv(pool, layer, tables[r], len(p))[kv]
                want = torch.cat([ref_pools[layer][kv][b] for b in tables[r]])[:len(p)].transpose(0, 1)
                assert_bits(got, want)
                want = torch.cat([cpu_pools[layer][kv][b] for b in tables[r]])[:len(p)].transpose(0, 1)
                assert_kv_near(got, want)


def test_mixed_step_matches_separate_chunk_and_decode_steps(models):
    """One forward over two prompt chunks (one with history, one completing its prompt) and three
    decoding requests: logits and stored K/V bit-identical to the oracle's mixed step (the same
    flattened batch: ragged chunk rows padded to 128 chunk tokens and 4 decode rows, as reference
    numerics run every mixed step), greedy tokens equal to the chunk step and the decode step run
    apart and to the CPU oracle, logits close to the decode step's."""
    model, ref, ref_cpu = models
    cfg = model.config
    runner = PagedRunner(model)
    decoders = prompts_of([45, 17, 3], seed=8)
    chunked = prompts_of([70, 20], seed=9)
    pools = [make_pool(cfg, 64), make_pool(cfg, 64)]
    ref_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, BS, 8, 128, device="cuda:0")
    cpu_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, BS, 8, 128)
    manager = KVCacheManager(BS, num_blocks=64)
    for i, p in enumerate(decoders + chunked):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(5)]
    # set-up, identical on both pools: decoders prefilled, request 3 has its first 30 tokens cached
    first = None
    for pool in pools:
        out = runner.run_prefill_step(decoders)
        runner.store_prefill(pool, out.prefill_cache, tables[:3], [len(p) for p in decoders], [0] * 3)
        part = runner.run_prefill_chunk_step([chunked[0][:30]], [0], [tables[3]], pool)
        runner.store_prefill(pool, part.prefill_cache, [tables[3]], [30], [0])
        first = out.next_tokens
    for oracle, opools in ((ref, ref_pools), (ref_cpu, cpu_pools)):
        _, presents = qwen3_ref.prefill(oracle, decoders)
        qwen3_ref.store_prefill(opools, presents, tables[:3], [len(p) for p in decoders], [0] * 3, BS)
        _, presents = qwen3_ref.prefill_chunk_step(oracle, [chunked[0][:30]], [0], [tables[3]], opools, BS)
        qwen3_ref.store_prefill(opools, presents, [tables[3]], [30], [0], BS)
    chunks, starts = [chunked[0][30:], chunked[1]], [30, 0]
    lens = [len(c) for c in chunks]
    positions = [len(p) for p in decoders]
    for i in range(3):
        assert manager.allocate_slots(i, 1)
    dec_tables = [manager.block_table(i) for i in range(3)]
    pf_tables = [tables[3], tables[4]]
    with torch.inference_mode():
        # apart: chunk step + store, then decode step (pool 0)
        apart = runner.run_prefill_chunk_step(chunks, starts, pf_tables, pools[0])
        runner.store_prefill(pools[0], apart.prefill_cache, pf_tables, lens, starts)
        ids, pos, meta = runner.prepare_decode_inputs(dec_tables, first, positions, BS)
        dec_logits = model(ids, position_ids=pos, attn_metadata=meta._replace(kv_pools=tuple(pools[0].kv_pools)),
                           last_logits_only=True)[0][:, -1].float()
        # mixed (pool 1)
        ids, pos, meta = runner.prepare_mixed_inputs(chunks, starts, pf_tables, first, positions, dec_tables,
                                                     pools[1])
        assert ids.shape == (1, 128 + 4)
        assert meta.live_decode_rows == 3 and meta.chunk_first_host == (0, lens[0])
        # the decode rows' append rewrites the same values when the step runs again
        mixed_logits = model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)[0][:5, -1]
        # another step prepared before this one runs leaves this one's rows and live decode rows alone
        runner.prepare_mixed_inputs(chunks[::-1], starts[::-1], pf_tables[::-1], first[:2], positions[:2],
                                    dec_tables[:2], pools[1])
        got = runner.run_mixed_step(ids, pos, meta)
        assert got.prefill_cache.ragged_first == [0, lens[0]] and len(got.decode_next_tokens) == 3
        # metadata without the host copy: the same first tokens from its device rows
        assert PagedRunner._ragged_cache(got.prefill_cache.past_key_values,
                                         meta._replace(chunk_first_host=None)).ragged_first == [0, lens[0]]
        runner.store_prefill(pools[1], got.prefill_cache, pf_tables, lens, starts)
    want_mixed, presents = qwen3_ref.mixed_step_logits(ref, chunks, starts, pf_tables, first, positions, dec_tables,
                                                       ref_pools, BS, chunk_tokens=128, decode_rows=4)
    qwen3_ref.store_prefill(ref_pools, presents, pf_tables, lens, starts, BS)
    assert torch.equal(mixed_logits, want_mixed)
    want_dec = qwen3_ref.decode_step(ref_cpu, dec_tables, first, positions, cpu_pools, BS)
    want_pf, _ = qwen3_ref.prefill_chunk_step(ref_cpu, chunks, starts, pf_tables, cpu_pools, BS)
    assert got.decode_next_tokens == dec_logits.argmax(-1).tolist() == want_dec.argmax(-1).tolist()
    assert got.prefill_next_tokens == apart.next_tokens == want_pf
    mixed_logits = mixed_logits.float()
    assert (mixed_logits[2:] - dec_logits).abs().max().item() <= LOGIT_RTOL * dec_logits.abs().max().item()
    for r in range(5):
        length = positions[r] + 1 if r < 3 else len(chunked[r - 3])
        table = manager.block_table(r)
        for layer in range(cfg.num_hidden_layers):
            for kv in range(2):
                a = request_kv(pools[0], layer, table, length)[kv]
                b = request_kv(pools[1], layer, table, length)[kv]
                assert_kv_close(layer, b, a)
                want = torch.cat([ref_pools[layer][kv][x] for x in table])[:length].transpose(0, 1)
                assert_bits(b, want)


def test_decode_graph_replays_match_eager_forward_and_touch_only_live_slots(fast_model):
    """Decode graphs over padded buckets (the bandwidth form): each replay equals an eager forward of
    the same padded inputs, bit for bit, with eager work and syncs between replays; pad rows write
    nothing; batches shrink and grow across buckets and contexts cross block boundaries."""
    model = fast_model
    cfg = model.config
    prompts = prompts_of([30, 17, 5, 44], seed=7)
    manager = KVCacheManager(BS, num_blocks=40)
    pool = make_pool(cfg, 40)
    runner = PagedRunner(model)
    runner.enable_decode_graphs(pool, max_batch=4, max_blocks=8, batch_buckets=[1, 2, 4])
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    out = runner.run_prefill_step(prompts)
    runner.store_prefill(pool, out.prefill_cache, [manager.block_table(i) for i in range(4)],
                         [len(p) for p in prompts], [0] * 4)
    tokens = {i: [t] for i, t in enumerate(out.next_tokens)}
    lengths = {i: len(p) for i, p in enumerate(prompts)}
    schedule = [[0, 1, 2, 3], [0, 1, 2], [0, 2], [2], [1, 3], [0, 1, 2, 3], [3, 1]]
    replays = 0
    with torch.inference_mode():
        for active in schedule:
            for i in active:
                assert manager.allocate_slots(i, 1)
            tables = [manager.block_table(i) for i in active]
            ids, pos, meta = runner.prepare_decode_inputs(tables, [tokens[i][-1] for i in active],
                                                          [lengths[i] for i in active], BS)
            graph = runner._loaded[0]
            assert graph.batch >= len(active) and meta.slot_mapping.data_ptr() == graph.static[:, 2].data_ptr()
            full_ids, full_pos, full_meta = graph.views(graph.batch)
            before = [t.clone() for kv in pool.kv_pools for t in kv]
            eager = model(full_ids, position_ids=full_pos,
                          attn_metadata=full_meta._replace(kv_pools=tuple(pool.kv_pools)),
                          last_logits_only=True)[0][:, -1]
            torch.cuda.synchronize()
            got = runner.run_decode_step(ids, pos, meta, pool)
            replays += 1
            assert torch.equal(graph.logits, eager), f"replay {replays} differs from the eager forward"
            assert got.next_tokens == eager[:len(active)].argmax(-1).tolist()
            live = set(meta.slot_mapping.tolist())
            after = [t for kv in pool.kv_pools for t in kv]
            for b, a in zip(before, after):
                changed = (b.view(-1, 8 * 128) != a.view(-1, 8 * 128)).any(dim=1).nonzero().flatten().tolist()
                assert set(changed) <= live
            for i, t in zip(active, got.next_tokens):
                tokens[i].append(t)
                lengths[i] += 1
    assert replays == len(schedule)


def test_exact_decode_graphs_per_batch_match_eager_and_oracle(models):
    """Reference numerics: one decode graph per batch size (no padded rows) and one table width;
    each replay bit-identical to the eager forward and to the oracle with the same numerics."""
    model, ref, _ = models
    cfg = model.config
    prompts = prompts_of([30, 17, 5, 44], seed=7)
    manager = KVCacheManager(BS, num_blocks=40)
    pool = make_pool(cfg, 40)
    ref_pools = torch_ref.make_pools(cfg.num_hidden_layers, 40, BS, 8, 128, device="cuda:0")
    runner = PagedRunner(model)
    runner.enable_decode_graphs(pool, max_batch=4, max_blocks=8)
    assert sorted(runner._graphs) == [(b, 8) for b in (1, 2, 3, 4)]
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(4)]
    out = runner.run_prefill_step(prompts)
    runner.store_prefill(pool, out.prefill_cache, tables, [len(p) for p in prompts], [0] * 4)
    first, presents = qwen3_ref.prefill(ref, prompts)
    qwen3_ref.store_prefill(ref_pools, presents, tables, [len(p) for p in prompts], [0] * 4, BS)
    assert out.next_tokens == first
    tokens = {i: [t] for i, t in enumerate(out.next_tokens)}
    lengths = {i: len(p) for i, p in enumerate(prompts)}
    with torch.inference_mode():
        for active in [[0, 1, 2, 3], [0, 1, 2], [0, 2], [2], [1, 3], [3, 1, 0]]:
            for i in active:
                assert manager.allocate_slots(i, 1)
            tables = [manager.block_table(i) for i in active]
            last, lens = [tokens[i][-1] for i in active], [lengths[i] for i in active]
            ids, pos, meta = runner.prepare_decode_inputs(tables, last, lens, BS)
            graph = runner._loaded[0]
            assert graph.batch == len(active)
            got = runner.run_decode_step(ids, pos, meta, pool)
            want = qwen3_ref.decode_step(ref, tables, last, lens, ref_pools, BS)
            assert torch.equal(graph.logits, want)
            assert got.next_tokens == want.float().argmax(-1).tolist()
            for i, t in zip(active, got.next_tokens):
                tokens[i].append(t)
                lengths[i] += 1


def test_exact_models_refuse_prefill_graphs_and_other_mixed_shapes(models):
    """Reference numerics: no prefill graphs (they pad the chunk width), and mixed graphs only at the
    shapes every mixed step runs at (width multiples of 128, power-of-two decode rows)."""
    model = models[0]
    runner = PagedRunner(model)
    pool = make_pool(model.config, 8)
    with pytest.raises(ValueError, match="pad the chunk width"):
        runner.enable_prefill_graphs(pool, max_rows=1, max_width=128, max_history_blocks=4)
    with pytest.raises(ValueError, match="power-of-two decode rows"):
        runner.enable_mixed_graphs(pool, max_rows=1, max_width=128, max_decode_rows=3, max_history_blocks=4,
                                   max_decode_blocks=4, decode_row_buckets=[3])
    with pytest.raises(ValueError, match="power-of-two decode rows"):
        runner.enable_mixed_graphs(pool, max_rows=1, max_width=128, max_decode_rows=2, max_history_blocks=4,
                                   max_decode_blocks=4, width_quantum=64)
    assert not runner._mixed_graphs


def test_exact_mixed_graph_replays_match_eager_runner_and_oracle(models):
    """Reference numerics run every mixed step at its padded shape (ragged chunk rows, their tokens
    rounded up to a multiple of 128, decode rows to a power of two), graphed or not: graph replays
    equal an eager forward of the same inputs, and the logits of both equal the GPU oracle's mixed
    step at that shape, bit for bit, with eager work and syncs between replays and one bucket
    replayed twice; steps outside the buckets (three chunk rows, a chunk longer than the graphs
    serve) run eagerly at the same padded shape.
    Tokens of the graphed and the eager runner are equal and the pools bit-identical to the
    oracle's."""
    model, ref, _ = models
    cfg = model.config
    decoders = prompts_of([45, 17, 3], seed=8)
    chunked = prompts_of([70, 20, 50, 33, 12, 9, 40, 130], seed=9)
    pools = [make_pool(cfg, 64), make_pool(cfg, 64)]  # graphed, eager
    ref_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, BS, 8, 128, device="cuda:0")
    manager = KVCacheManager(BS, num_blocks=64)
    graphed, eager_runner = PagedRunner(model), PagedRunner(model)
    graphed.enable_mixed_graphs(pools[0], max_rows=2, max_width=128, max_decode_rows=4, max_history_blocks=8,
                                max_decode_blocks=8)
    assert sorted(graphed._mixed_graphs) == sorted([(1, 128, d) for d in (1, 2, 4)] +
                                                   [(2, c, d) for c in (128, 256) for d in (1, 2, 4)])
    n_req = len(decoders) + len(chunked)
    for i, p in enumerate(decoders + chunked):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(n_req)]
    with torch.inference_mode():
        for pool, runner in zip(pools, (graphed, eager_runner)):
            out = runner.run_prefill_step(decoders)
            runner.store_prefill(pool, out.prefill_cache, tables[:3], [len(p) for p in decoders], [0] * 3)
    _, presents = qwen3_ref.prefill(ref, decoders)
    qwen3_ref.store_prefill(ref_pools, presents, tables[:3], [len(p) for p in decoders], [0] * 3, BS)
    last, positions = list(out.next_tokens), [len(p) for p in decoders]
    # (chunks as (chunked request, start, end), decoding requests, replayed from a graph)
    steps = [([(0, 0, 30)], [0, 1, 2], True), ([(0, 30, 70), (1, 0, 20)], [0, 1, 2], True),
             ([(2, 0, 50)], [0, 2], True), ([(3, 0, 33), (4, 0, 12), (5, 0, 9)], [0, 1], False),
             ([(6, 0, 40)], [0, 1, 2], True), ([(7, 0, 130)], [1], False)]
    replays = 0
    with torch.inference_mode():
        for chunks, dec, graphed_step in steps:
            for i in dec:
                assert manager.allocate_slots(i, 1)
            dec_tables = [manager.block_table(i) for i in dec]
            chunk_ids = [chunked[c][a:b] for c, a, b in chunks]
            starts, lens = [a for _, a, _ in chunks], [b - a for _, a, b in chunks]
            pf_tables = [tables[3 + c] for c, _, _ in chunks]
            chunk_tokens, dec_rows = -(-sum(lens) // 128) * 128, 1 << (len(dec) - 1).bit_length()
            live = len(chunks) + len(dec)
            results = []
            for pool, runner in zip(pools, (graphed, eager_runner)):
                ids, pos, meta = runner.prepare_mixed_inputs(chunk_ids, starts, pf_tables, [last[i] for i in dec],
                                                             [positions[i] for i in dec], dec_tables, pool)
                assert ids.shape == (1, chunk_tokens + dec_rows)
                replayed = runner is graphed and runner._mixed_loaded is not None
                assert replayed == (graphed_step and runner is graphed)
                eager, eager_present = model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
                torch.cuda.synchronize()
                got = runner.run_mixed_step(ids, pos, meta)
                if replayed:
                    replays += 1
                    graph = runner._mixed_loaded[0]
                    assert torch.equal(graph.logits, eager[:, -1]), f"replay {replays} differs from the eager forward"
                    for (k, v), (ek, ev) in zip(got.prefill_cache, eager_present):
                        assert torch.equal(k, ek) and torch.equal(v, ev)
                runner.store_prefill(pool, got.prefill_cache, pf_tables, lens, starts)
                results.append((got, eager[:live, -1].clone()))
            want, presents = qwen3_ref.mixed_step_logits(ref, chunk_ids, starts, pf_tables, [last[i] for i in dec],
                                                         [positions[i] for i in dec], dec_tables, ref_pools, BS,
                                                         chunk_tokens=chunk_tokens, decode_rows=dec_rows)
            qwen3_ref.store_prefill(ref_pools, presents, pf_tables, lens, starts, BS)
            for got, logits in results:
                assert torch.equal(logits, want)
                assert got.decode_next_tokens == want[len(chunks):].float().argmax(-1).tolist()
                assert got.prefill_next_tokens == want[:len(chunks)].float().argmax(-1).tolist()
            for i, t in zip(dec, results[0][0].decode_next_tokens):
                last[i], positions[i] = t, positions[i] + 1
    assert replays == 4
    torch.cuda.synchronize()
    assert_bits(pools[0].storage, pools[1].storage)
    for r in range(n_req):
        length = positions[r] if r < 3 else len(chunked[r - 3])
        table = manager.block_table(r)
        for layer in range(cfg.num_hidden_layers):
            for kv in range(2):
                want = torch.cat([ref_pools[layer][kv][x] for x in table])[:length].transpose(0, 1)
                assert_bits(request_kv(pools[0], layer, table, length)[kv], want)


@pytest.mark.parametrize("form", ["exact_eager", "bandwidth_graphs"])
def test_prefill_direct_pool_write_matches_the_two_pass_store(models, fast_model, form):
    """When the block tables already cover the chunk, q/k norm + RoPE writes the chunk's K/V rows
    straight into their slots and store_prefill finds nothing left to do; the pools are then
    bit-identical to the two-pass path (tables covering only the history during the forward, the
    scatter afterwards).  Reference numerics eagerly, and the bandwidth form through prefill graphs."""
    model = models[0] if form == "exact_eager" else fast_model
    cfg = model.config
    prompts = prompts_of([70, 45, 100], seed=21)
    manager = KVCacheManager(BS, num_blocks=48)
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(3)]
    pools = [make_pool(cfg, 48), make_pool(cfg, 48)]  # direct, two-pass
    runners = [PagedRunner(model), PagedRunner(model)]
    if form == "bandwidth_graphs":
        for runner, pool in zip(runners, pools):
            runner.enable_prefill_graphs(pool, max_rows=3, max_width=128, max_history_blocks=8)
    steps = [([0, 1, 2], [0, 0, 0], [40, 20, 64]), ([0, 1, 2], [40, 20, 64], [70, 45, 100])]
    with torch.inference_mode():
        for reqs, starts, ends in steps:
            chunks = [prompts[r][s:e] for r, s, e in zip(reqs, starts, ends)]
            lens = [e - s for s, e in zip(starts, ends)]
            full = [tables[r] for r in reqs]
            history_only = [t[:-(-s // BS)] for t, s in zip(full, starts)]
            direct = runners[0].run_prefill_chunk_step(chunks, starts, full, pools[0])
            assert direct.prefill_cache.written_index is not None
            runners[0].store_prefill(pools[0], direct.prefill_cache, full, lens, starts)
            two_pass = runners[1].run_prefill_chunk_step(chunks, starts, history_only, pools[1])
            assert two_pass.prefill_cache.written_index is None
            runners[1].store_prefill(pools[1], two_pass.prefill_cache, full, lens, starts)
            assert direct.next_tokens == two_pass.next_tokens
            torch.cuda.synchronize()
            assert_bits(pools[0].storage, pools[1].storage)
    for r, p in enumerate(prompts):  # every token of every prompt is in place
        assert request_kv(pools[0], 0, tables[r], len(p))[0].abs().sum() > 0


def test_prefill_graph_replays_match_eager_forward(fast_model, models):
    """Prefill graphs: each replay equals an eager forward of the same padded inputs, bit for bit
    (logits and the chunk K/V), with eager work and syncs between replays, across row counts, widths
    and history buckets; the tokens and stored K/V equal the eager runner's (which pads the chunk to
    its own width, so values agree to rounding) and the CPU oracle's tokens.  Bandwidth form."""
    model, ref_cpu = fast_model, models[2]
    cfg = model.config
    prompts = prompts_of([150, 90, 60, 200, 300], seed=12)
    manager = KVCacheManager(BS, num_blocks=64)
    pools = [make_pool(cfg, 64), make_pool(cfg, 64)]  # graphed, eager
    cpu_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, BS, 8, 128)
    graphed, eager_runner = PagedRunner(model), PagedRunner(model)
    graphed.enable_prefill_graphs(pools[0], max_rows=2, max_width=256, max_history_blocks=16)
    assert len(graphed._prefill_graphs) == 2 * 2
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(5)]
    # (requests, chunk starts, chunk ends): no history, two rows, two rows with history, the first
    # bucket again, a history of 100 tokens (7 blocks), and a chunk too wide for the buckets (eager)
    steps = [([0], [0], [70]), ([1, 2], [0, 0], [40, 60]), ([0, 1], [70, 40], [150, 90]), ([3], [0], [100]),
             ([3], [100], [200]), ([4], [0], [300])]
    replays = 0
    with torch.inference_mode():
        for reqs, starts, ends in steps:
            chunks = [prompts[r][s:e] for r, s, e in zip(reqs, starts, ends)]
            tabs = [tables[r] for r in reqs]
            lens = [e - s for s, e in zip(starts, ends)]
            got = graphed.run_prefill_chunk_step(chunks, starts, tabs, pools[0])
            graph = graphed._prefill_bucket(len(reqs), max(lens), -(-max(starts) // BS))
            if graph is not None:
                replays += 1
                ids, pos, meta = graph.views()
                logits = graph.logits.clone()
                present = [(k.clone(), v.clone()) for k, v in got.prefill_cache]
                eager, eager_present = model(ids, position_ids=pos, last_logits_only=True,
                                             attn_metadata=meta._replace(kv_pools=tuple(pools[0].kv_pools)))
                torch.cuda.synchronize()
                assert torch.equal(logits, eager[:, -1]), f"replay {replays} differs from the eager forward"
                for (k, v), (ek, ev) in zip(present, eager_present):
                    assert torch.equal(k, ek) and torch.equal(v, ev)
            want = eager_runner.run_prefill_chunk_step(chunks, starts, tabs, pools[1])
            graphed.store_prefill(pools[0], got.prefill_cache, tabs, lens, starts)
            eager_runner.store_prefill(pools[1], want.prefill_cache, tabs, lens, starts)
            toks, presents = qwen3_ref.prefill_chunk_step(ref_cpu, chunks, starts, tabs, cpu_pools, BS)
            qwen3_ref.store_prefill(cpu_pools, presents, tabs, lens, starts, BS)
            assert got.next_tokens == want.next_tokens == toks
    assert replays == 5
    for r, p in enumerate(prompts):
        for layer in range(cfg.num_hidden_layers):
            for kv in range(2):
                assert_kv_close(layer, request_kv(pools[0], layer, tables[r], len(p))[kv],
                                request_kv(pools[1], layer, tables[r], len(p))[kv])


def test_mixed_graph_replays_match_eager_forward(fast_model, models):
    """Mixed graphs: each replay equals an eager forward of the same padded inputs, bit for bit
    (logits and chunk K/V), across chunk-row and decode-row buckets (pad decode rows write nothing);
    tokens equal the eager runner's unpadded mixed step and the CPU oracle's, stored K/V agree.
    Bandwidth form."""
    model, ref_cpu = fast_model, models[2]
    cfg = model.config
    decoders = prompts_of([45, 17, 3], seed=8)
    chunked = prompts_of([70, 20, 50], seed=9)
    pools = [make_pool(cfg, 64), make_pool(cfg, 64)]  # graphed, eager
    cpu_pools = torch_ref.make_pools(cfg.num_hidden_layers, 64, BS, 8, 128)
    manager = KVCacheManager(BS, num_blocks=64)
    graphed, eager_runner = PagedRunner(model), PagedRunner(model)
    graphed.enable_mixed_graphs(pools[0], max_rows=2, max_width=128, max_decode_rows=4, max_history_blocks=8,
                                max_decode_blocks=8, decode_row_buckets=[2, 4])
    assert len(graphed._mixed_graphs) == (1 + 2) * 2  # chunk tokens 128 (one row), 128 / 256 (two); 2 decode buckets
    for i, p in enumerate(decoders + chunked):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(6)]
    with torch.inference_mode():
        for pool, runner in zip(pools, (graphed, eager_runner)):
            out = runner.run_prefill_step(decoders)
            runner.store_prefill(pool, out.prefill_cache, tables[:3], [len(p) for p in decoders], [0] * 3)
    _, presents = qwen3_ref.prefill(ref_cpu, decoders)
    qwen3_ref.store_prefill(cpu_pools, presents, tables[:3], [len(p) for p in decoders], [0] * 3, BS)
    last, positions = list(out.next_tokens), [len(p) for p in decoders]
    # (chunks as (chunked request, start, end), decoding requests)
    steps = [([(0, 0, 30)], [0, 1, 2]), ([(0, 30, 70), (1, 0, 20)], [0, 1, 2]), ([(2, 0, 50)], [0, 2])]
    with torch.inference_mode():
        for chunks, dec in steps:
            for i in dec:
                assert manager.allocate_slots(i, 1)
            dec_tables = [manager.block_table(i) for i in dec]
            chunk_ids = [chunked[c][a:b] for c, a, b in chunks]
            starts, lens = [a for _, a, _ in chunks], [b - a for _, a, b in chunks]
            pf_tables = [tables[3 + c] for c, _, _ in chunks]
            results = []
            for pool, runner in zip(pools, (graphed, eager_runner)):
                ids, pos, meta = runner.prepare_mixed_inputs(chunk_ids, starts, pf_tables, [last[i] for i in dec],
                                                             [positions[i] for i in dec], dec_tables, pool)
                if runner is graphed:
                    graph = runner._mixed_loaded[0]
                    assert graph.rows == len(chunks) and graph.decode_rows >= len(dec)
                    eager, eager_present = model(ids, position_ids=pos, attn_metadata=meta, last_logits_only=True)
                    torch.cuda.synchronize()
                got = runner.run_mixed_step(ids, pos, meta)
                if runner is graphed:
                    assert torch.equal(graph.logits, eager[:, -1])
                    for (k, v), (ek, ev) in zip(got.prefill_cache, eager_present):
                        assert torch.equal(k, ek) and torch.equal(v, ev)
                runner.store_prefill(pool, got.prefill_cache, pf_tables, lens, starts)
                results.append(got)
            want_dec = qwen3_ref.decode_step(ref_cpu, dec_tables, [last[i] for i in dec], [positions[i] for i in dec],
                                             cpu_pools, BS)
            want_pf, presents = qwen3_ref.prefill_chunk_step(ref_cpu, chunk_ids, starts, pf_tables, cpu_pools, BS)
            qwen3_ref.store_prefill(cpu_pools, presents, pf_tables, lens, starts, BS)
            assert results[0].decode_next_tokens == results[1].decode_next_tokens == want_dec.argmax(-1).tolist()
            done = [k for k, (c, _, b) in enumerate(chunks) if b == len(chunked[c])]
            assert [results[0].prefill_next_tokens[k] for k in done] == \
                [results[1].prefill_next_tokens[k] for k in done] == [want_pf[k] for k in done]
            for i, t in zip(dec, results[0].decode_next_tokens):
                last[i], positions[i] = t, positions[i] + 1
    for r in range(6):
        length = positions[r] if r < 3 else len(chunked[r - 3])
        for layer in range(cfg.num_hidden_layers):
            for kv in range(2):
                assert_kv_close(layer, request_kv(pools[0], layer, tables[r], length)[kv],
                                request_kv(pools[1], layer, tables[r], length)[kv])


def test_decode_from_persistent_device_tables_matches_the_packed_path(models):
    """prepare_decode_from_tables (block tables kept on the GPU, updated by deltas; [B, 5] per step)
    gives the logits of prepare_decode_inputs (the reference's [B, 4 + max_blocks] packing), bit for
    bit, eagerly and through per-batch decode graphs, as requests grow across block boundaries,
    finish and are replaced."""
    from mini_infra_qwen3_amd.worker import DeviceBlockTables

    model = models[0]
    cfg = model.config
    prompts = prompts_of([30, 17, 5, 44, 23], seed=21)
    manager = KVCacheManager(BS, num_blocks=64)
    pool = make_pool(cfg, 64)
    tables = DeviceBlockTables(manager, max_rows=4, max_blocks=8, device="cuda:0")
    graphed = PagedRunner(model)
    graphed.enable_decode_graphs(pool, max_batch=4, max_blocks=8, tables=tables)
    eager = PagedRunner(model)
    for i, p in enumerate(prompts[:4]):
        manager.allocate_slots(i, len(p))
    out = eager.run_prefill_step(prompts[:4])
    eager.store_prefill(pool, out.prefill_cache, [manager.block_table(i) for i in range(4)],
                        [len(p) for p in prompts[:4]], [0] * 4)
    tokens = {i: [t] for i, t in enumerate(out.next_tokens)}
    lengths = {i: len(p) for i, p in enumerate(prompts)}
    schedule = [[0, 1, 2, 3]] * 3 + [[0, 2, 3]] * 2 + [[0, 2, 3, 4]] * 4 + [[4, 2]] * 3
    with torch.inference_mode():
        for active in schedule:
            if 4 in active and 4 not in tokens:  # request 1 finished: request 4 takes its row
                manager.free(1)
                manager.allocate_slots(4, len(prompts[4]))
                first = eager.run_prefill_step([prompts[4]])
                eager.store_prefill(pool, first.prefill_cache, [manager.block_table(4)], [len(prompts[4])], [0])
                tokens[4] = list(first.next_tokens)
            for i in active:
                assert manager.allocate_slots(i, 1)
            last, lens = [tokens[i][-1] for i in active], [lengths[i] for i in active]
            ids, pos, meta = eager.prepare_decode_inputs([manager.block_table(i) for i in active], last, lens, BS)
            want = model(ids, position_ids=pos, attn_metadata=meta._replace(kv_pools=tuple(pool.kv_pools)),
                         last_logits_only=True)[0][:, -1]
            ids, pos, meta = eager.prepare_decode_from_tables(tables, active, last, lens)
            got = model(ids, position_ids=pos, attn_metadata=meta._replace(kv_pools=tuple(pool.kv_pools)),
                        last_logits_only=True)[0][:, -1]
            assert torch.equal(got, want)
            ids, pos, meta = graphed.prepare_decode_from_tables(tables, active, last, lens)
            assert graphed._loaded is not None and graphed._loaded[0].batch == len(active)
            step = graphed.run_decode_step(ids, pos, meta, pool)
            assert torch.equal(graphed._loaded[0].logits, want)
            assert step.next_tokens == want.float().argmax(-1).tolist()
            for i, t in zip(active, step.next_tokens):
                tokens[i].append(t)
                lengths[i] += 1
