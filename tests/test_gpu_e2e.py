"""Continuous batching with chunked prefill on Qwen3-0.6B (28 layers, hidden 1024, vocab 151936,
bf16, random init): the HIP model against the oracle's restatement of the reference torch path with
exact sums (``ReferenceQwen3(exact=True)``, on cuda:0 with the same weights and the same GEMM
calls), both driven through the same scheduler loop with a fixed logical step clock, so that they
execute the identical step sequence.  Both run free: each feeds back its own greedy tokens.

The bar is the reference's own correctness gate, exact token equality
(src/mini_infra/bench/correctness.py:69-73): every request's generated sequence must be identical.
The logits are bit-identical, so even exact bf16 ties (common over 151,936 tokens) resolve to the
same first index on both sides and no divergence is tolerated; a failure prints each request's
first divergence with the oracle's logit gap there.
"""

import pytest
import torch

from mini_infra_qwen3_amd.core.scheduler import SchedulePhase
from mini_infra_qwen3_amd.engine import PagedScheduleBackend, run_scheduler
from mini_infra_qwen3_amd.model import Qwen3ForCausalLM, init_random_, qwen3_0_6b
from mini_infra_qwen3_amd.workloads import serving_requests
from oracle import qwen3_ref

pytestmark = pytest.mark.gpu


def step_clock(out):
    return {SchedulePhase.PREFILL: 10.0, SchedulePhase.MIXED: 12.0}.get(out.phase, 5.0)


def build(untied_head_seed=None):
    cfg = qwen3_0_6b()
    model = Qwen3ForCausalLM(cfg)
    init_random_(model, seed=0, std=0.02, untied_head_seed=untied_head_seed)
    model = model.to(torch.bfloat16)
    weights = {k: v.clone() for k, v in model.state_dict().items()}
    return model.to("cuda:0").eval(), qwen3_ref.ReferenceQwen3(cfg, weights, "cuda:0", exact=True)


def compare(product, oracle, backend):
    """Per request: identical, or the first divergence and the oracle's logit gap there."""
    assert [(e.phase, e.request_ids, e.chunk_spans) for e in product.events] == \
        [(e.phase, e.request_ids, e.chunk_spans) for e in oracle.events]
    gaps = {(r, k): gap for r, k, _, _, gap, _ in backend.records}
    diverged = {}
    for r, tokens in product.tokens.items():
        want = oracle.tokens[r]
        assert len(tokens) == len(want)
        k = next((i for i, (a, b) in enumerate(zip(tokens, want)) if a != b), None)
        if k is not None:
            diverged[r] = (k, tokens[k], want[k], gaps[(r, k)])
    print(f"\n{len(product.tokens) - len(diverged)} of {len(product.tokens)} requests identical; first divergences "
          f"(request: index, HIP token, oracle token, oracle logit gap): {diverged}")
    return diverged


@pytest.mark.timeout(900)
@pytest.mark.parametrize("mixed,chunk_cap", [(False, None), (True, None), (True, 1024)],
                         ids=["alternating", "mixed_batching", "mixed_batching_chunk_cap"])
def test_continuous_batching_run_greedy_tokens_identical_to_the_oracle(mixed, chunk_cap):
    """The full workload: 128 requests, Poisson arrivals at 20 req/s, prompts U[32, 1024], 128 greedy
    tokens each, token budget 2048, 128 batch slots; decode steps replay HIP graphs.  The mixed runs
    (the bench's reference-numerics mixed legs) replay mixed graphs at the padded step shapes, the
    last with at most 1024 prompt tokens per mixed step."""
    model, ref = build()
    requests = serving_requests(seed=0)
    assert len(requests) == 128 and all(r.max_new_tokens == 128 for r in requests)
    backend = PagedScheduleBackend(model, requests, 128, decode_graphs=True, mixed_graphs=mixed,
                                   mixed_graph_tokens=chunk_cap or 2048)
    product = run_scheduler(backend, requests, token_budget=2048, max_running_requests=128, eos_token_id=-1,
                            stop_on_eos=False, step_clock=step_clock, mixed_batching=mixed,
                            mixed_chunk_tokens=chunk_cap)
    if mixed:
        assert product.num_steps(SchedulePhase.MIXED) > 100 and product.num_steps(SchedulePhase.DECODE) > 1000
    else:
        assert product.num_steps(SchedulePhase.PREFILL) > 100 and product.num_steps(SchedulePhase.DECODE) > 1000
    oracle_backend = qwen3_ref.ReferenceScheduleBackend(ref, requests, 128, watch_tokens=product.tokens)
    oracle = run_scheduler(oracle_backend, requests, token_budget=2048, max_running_requests=128, eos_token_id=-1,
                           stop_on_eos=False, step_clock=step_clock, mixed_batching=mixed,
                           mixed_chunk_tokens=chunk_cap)
    assert len(oracle_backend.records) == 128 * 128
    diverged = compare(product, oracle, oracle_backend)
    assert not diverged, diverged


@pytest.mark.timeout(600)
@pytest.mark.parametrize("untied_head_seed,mixed,chunk_cap", [(1234, False, None), (None, True, None), (None, True, 96)],
                         ids=["context_dependent_model", "mixed_batching", "mixed_batching_chunk_cap"])
def test_greedy_tokens_identical_on_chunked_slices(untied_head_seed, mixed, chunk_cap):
    """24 requests with prompts up to 700 tokens and 48 outputs under a 256-token budget, so that
    prompts are chunked over several steps with history.  ``context_dependent_model``: an untied
    N(0, 1) head (output that depends on the whole context, as the reference's diverse test model:
    tests/unit/conftest.py:13-25).  ``mixed_batching``: decode rows and prompt chunks share steps,
    replayed from mixed graphs where a bucket fits (the oracle runs a mixed step as one forward over
    the same flattened batch, padded to the same shape).  ``mixed_batching_chunk_cap``: at most 96
    prompt tokens in a mixed step (prefill-only steps keep the budget)."""
    model, ref = build(untied_head_seed)
    requests = serving_requests(seed=1, num_requests=24, min_prompt=32, max_prompt=700, max_new_tokens=48)
    mrr, budget = 8, 256
    backend = PagedScheduleBackend(model, requests, mrr, decode_graphs=True, mixed_graphs=mixed,
                                   mixed_graph_tokens=chunk_cap or budget)
    product = run_scheduler(backend, requests, token_budget=budget, max_running_requests=mrr, eos_token_id=-1,
                            stop_on_eos=False, step_clock=step_clock, mixed_batching=mixed,
                            mixed_chunk_tokens=chunk_cap)
    chunk_steps = product.num_steps(SchedulePhase.PREFILL) + product.num_steps(SchedulePhase.MIXED)
    assert chunk_steps > len(requests)  # prompts were chunked
    assert (product.num_steps(SchedulePhase.MIXED) > 0) == mixed
    if chunk_cap:
        assert max(sum(b - a for a, b in e.chunk_spans) for e in product.events
                   if e.phase is SchedulePhase.MIXED) <= chunk_cap
    oracle_backend = qwen3_ref.ReferenceScheduleBackend(ref, requests, mrr, watch_tokens=product.tokens)
    oracle = run_scheduler(oracle_backend, requests, token_budget=budget, max_running_requests=mrr, eos_token_id=-1,
                           stop_on_eos=False, step_clock=step_clock, mixed_batching=mixed,
                           mixed_chunk_tokens=chunk_cap)
    diverged = compare(product, oracle, oracle_backend)
    assert not diverged, diverged
