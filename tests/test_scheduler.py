"""Chunked-prefill iteration scheduler and the continuous-batching loop on the CPU.

Scheduler trajectories restate the reference's known answers (tests/unit/test_scheduler.py:498-640);
the loop invariants are those of tests/unit/test_paged_scheduler.py:338-360, checked with a
deterministic fake backend (no model, no device)."""

import pytest

from mini_infra_qwen3_amd.core import KVCacheManager, Request
from mini_infra_qwen3_amd.core.scheduler import IterationScheduler, RequestState, SchedulePhase
from mini_infra_qwen3_amd.engine import ScheduleStepOutput, percentile, run_scheduler

DECODE, PREFILL, MIXED = SchedulePhase.DECODE, SchedulePhase.PREFILL, SchedulePhase.MIXED


def states_with(prompt_lens, max_new=4):
    return [RequestState(Request(i, tuple(range(1, n + 1)), max_new)) for i, n in enumerate(prompt_lens)]


def scheduler(token_budget, capacity, manager=None, mixed=False, mixed_chunk_tokens=None):
    return IterationScheduler(token_budget, capacity, manager or KVCacheManager(4, 1000), mixed=mixed,
                              mixed_chunk_tokens=mixed_chunk_tokens)


def ranges(out):
    return [(c.state.request.request_idx, c.start, c.end) for c in out.prefill_chunks]


def step(sched, clock):
    out = sched.schedule(clock)
    assert out is not None
    n = sum(c.is_last for c in out.prefill_chunks) + len(out.decode_requests)
    sched.update_from_output(out, [7] * n, clock, stop_on_eos=False)
    return out


def test_splits_prompts_with_shared_budget():
    s = scheduler(8, 4)
    s.add_requests(states_with([10, 10, 3]))
    first = step(s, 0.0)
    assert ranges(first) == [(0, 0, 2), (1, 0, 2), (2, 0, 2)] and first.num_scheduled_tokens == 6
    assert not s.waiting and len(s.running) == 3
    assert ranges(step(s, 1.0)) == [(0, 2, 4), (1, 2, 4), (2, 2, 3)]
    decode = step(s, 2.0)
    assert decode.phase is DECODE and [st.request.request_idx for st in decode.scheduled_requests] == [2]
    third = step(s, 3.0)
    assert ranges(third) == [(0, 4, 8), (1, 4, 8)] and third.num_scheduled_tokens == 8


def test_decode_protection_alternates_prefill_and_decode():
    s = scheduler(4, 2)
    s.add_requests(states_with([2, 12], max_new=20))
    phases = [step(s, float(t)).phase for t in range(6)]
    assert phases == [PREFILL, DECODE, PREFILL, DECODE, PREFILL, DECODE]


def test_consecutive_prefill_without_decoders():
    s = scheduler(3, 1)
    s.add_requests(states_with([7]))
    assert ranges(step(s, 0.0)) == [(0, 0, 3)]
    assert ranges(step(s, 1.0)) == [(0, 3, 6)]
    third = step(s, 2.0)
    assert ranges(third) == [(0, 6, 7)] and third.prefill_chunks[0].is_last


def test_hard_budget_and_every_prompt_covered_once():
    lens = [17, 3, 9, 1, 25, 6, 12]
    s = scheduler(7, 4)
    s.add_requests(states_with(lens))
    covered = {i: [] for i in range(len(lens))}
    for t in range(200):
        if not s.has_unfinished_requests:
            break
        out = step(s, float(t))
        if out.phase is PREFILL:
            assert out.num_scheduled_tokens <= 7
            assert out.num_scheduled_tokens == len(out.prefill_chunks) * max(c.num_tokens for c in out.prefill_chunks)
            for c in out.prefill_chunks:
                covered[c.state.request.request_idx].append((c.start, c.end))
    assert not s.has_unfinished_requests
    for i, spans in covered.items():
        assert spans[0][0] == 0 and spans[-1][1] == lens[i]
        assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))


def test_partial_chunk_produces_no_token():
    s = scheduler(2, 2)
    states = states_with([5])
    s.add_requests(states)
    out = s.schedule(0.0)
    assert ranges(out) == [(0, 0, 2)] and states[0].cache_length == 0 and states[0].is_prefilling
    assert s.update_from_output(out, [], 1.0) == []
    assert states[0].cache_length == 2 and states[0].generated == [] and states[0].first_token_ms is None
    step(s, 1.0)
    last = s.schedule(2.0)
    assert last.prefill_chunks[0].is_last
    s.update_from_output(last, [9], 3.0, stop_on_eos=False)
    assert not states[0].is_prefilling and states[0].generated == [9] and states[0].first_token_ms == 3.0
    assert states[0].cache_length == 5


def test_allocates_blocks_per_chunk():
    manager = KVCacheManager(4, 8)
    s = scheduler(6, 2, manager)
    s.add_requests(states_with([10]))
    step(s, 0.0)
    assert manager.num_used_blocks == 2
    step(s, 1.0)
    assert manager.num_used_blocks == 3 and len(manager.block_table(0)) == 3


def test_admission_reserves_blocks_of_in_flight_prompts():
    manager = KVCacheManager(4, 6)
    s = scheduler(4, 4, manager)
    s.add_requests(states_with([12, 12]))
    assert ranges(step(s, 0.0)) == [(0, 0, 4)] and manager.num_used_blocks == 1
    assert ranges(step(s, 1.0)) == [(0, 4, 8)] and len(s.waiting) == 1
    assert ranges(step(s, 2.0)) == [(0, 8, 12)] and manager.num_used_blocks == 3 and len(s.waiting) == 1


def test_rejects_budget_below_capacity():
    with pytest.raises(ValueError):
        IterationScheduler(3, 4, KVCacheManager(4, 10))


def test_out_of_blocks_raises():
    s = scheduler(64, 2, KVCacheManager(4, 3))
    s.add_requests(states_with([8]))
    step(s, 0.0)
    with pytest.raises(RuntimeError):
        step(s, 1.0)


class FakeBackend:
    """Token = (request_idx * 31 + position) % 97 + 1, fixed step costs."""

    def __init__(self, block_size=4, num_blocks=200):
        self.kv_cache_manager = KVCacheManager(block_size, num_blocks)
        self.executed = []

    def execute_prefill(self, chunks):
        self.executed.append(("prefill", [(c.state.request.request_idx, c.start, c.end) for c in chunks]))
        toks = [(c.state.request.request_idx * 31 + c.end) % 97 + 1 for c in chunks if c.is_last]
        return ScheduleStepOutput(toks, 2.0, 0.5, len(chunks), 0)

    def execute_decode(self, states):
        self.executed.append(("decode", [s.request.request_idx for s in states]))
        toks = [(s.request.request_idx * 31 + s.cache_length + 1) % 97 + 1 for s in states]
        return ScheduleStepOutput(toks, 1.0, 0.25, len(states), 0)

    def execute_mixed(self, states, chunks):
        self.executed.append(("mixed", [s.request.request_idx for s in states],
                              [(c.state.request.request_idx, c.start, c.end) for c in chunks]))
        toks = [(s.request.request_idx * 31 + s.cache_length + 1) % 97 + 1 for s in states]
        toks += [(c.state.request.request_idx * 31 + c.end) % 97 + 1 for c in chunks if c.is_last]
        return ScheduleStepOutput(toks, 2.2, 0.6, len(states) + len(chunks), 0)


@pytest.mark.parametrize("budget,capacity", [(8, 2), (16, 4), (64, 8)])
def test_loop_invariants_and_metric(budget, capacity):
    lens, outs = [13, 4, 9, 2, 16, 30, 7], [5, 7, 3, 6, 4, 2, 9]
    arrivals = [0.0, 0.0, 3.0, 3.5, 20.0, 21.0, 200.0]
    requests = [Request(i, tuple(range(1, n + 1)), m, a) for i, (n, m, a) in enumerate(zip(lens, outs, arrivals))]
    backend = FakeBackend()
    result = run_scheduler(backend, requests, token_budget=budget, max_running_requests=capacity)
    assert [len(result.tokens[i]) for i in range(7)] == outs
    for i, n in enumerate(lens):  # every request decodes positions n, n+1, ... in order
        assert result.tokens[i][1:] == [(i * 31 + n + k + 1) % 97 + 1 for k in range(outs[i] - 1)]
    assert result.busy_ms == pytest.approx(sum(e.step_ms for e in result.events))
    assert result.throughput_tok_s == pytest.approx(sum(outs) * 1000 / result.busy_ms)
    for prev, cur in zip(result.events, result.events[1:]):
        if prev.phase is PREFILL and cur.phase is PREFILL:  # decode protection: no decoder was left
            assert prev.num_generated_tokens == len(prev.finished_request_ids)
    assert all(e.num_scheduled_tokens <= budget for e in result.events if e.phase is PREFILL)
    assert sorted(i for e in result.events for i in e.admitted_request_ids) == list(range(7))
    assert sorted(i for e in result.events for i in e.finished_request_ids) == list(range(7))
    assert max(len(e.request_ids) for e in result.events) <= capacity
    assert backend.kv_cache_manager.num_used_blocks == 0
    # an idle gap before the last arrival is not busy time
    assert result.makespan_ms > result.busy_ms


def test_loop_freezes_the_collector_only_while_it_runs():
    """The loop keeps the objects that exist when it starts out of cyclic collections while it runs
    and restores the collector afterwards, also when a step raises; with the collector disabled it
    leaves it alone."""
    import gc

    seen = []

    class Probe(FakeBackend):
        def execute_decode(self, states):
            seen.append((gc.isenabled(), gc.get_freeze_count() > 0))
            return super().execute_decode(states)

    class Failing(FakeBackend):
        def execute_prefill(self, chunks):
            raise RuntimeError("step failed")

    requests = [Request(i, tuple(range(1, 6)), 3, 0.0) for i in range(3)]
    assert gc.get_freeze_count() == 0
    run_scheduler(Probe(), requests, token_budget=16, max_running_requests=3)
    assert seen and all(enabled and frozen for enabled, frozen in seen)
    assert gc.isenabled() and gc.get_freeze_count() == 0
    with pytest.raises(RuntimeError, match="step failed"):
        run_scheduler(Failing(), requests, token_budget=16, max_running_requests=3)
    assert gc.isenabled() and gc.get_freeze_count() == 0
    seen.clear()
    gc.disable()
    try:
        run_scheduler(Probe(), requests, token_budget=16, max_running_requests=3)
    finally:
        gc.enable()
    assert seen and not any(frozen for _, frozen in seen)


def test_step_clock_makes_the_schedule_timing_independent():
    requests = [Request(i, tuple(range(1, 9 + 3 * i)), 4, 10.0 * i) for i in range(6)]
    a, b = FakeBackend(), FakeBackend()
    run_scheduler(a, requests, token_budget=8, max_running_requests=3, step_clock=lambda out: 5.0)
    run_scheduler(b, requests, token_budget=8, max_running_requests=3, step_clock=lambda out: 5.0)
    assert a.executed == b.executed


def test_mixed_steps_decode_while_prefilling():
    """Mixed batching (the reference's planned policy, core/scheduler.py:310-311): decoding requests
    take one token of the budget each, chunks share the rest, in one MIXED step."""
    s = scheduler(8, 4, mixed=True)
    s.add_requests(states_with([2, 20], max_new=10))
    first = step(s, 0.0)
    assert first.phase is PREFILL and ranges(first) == [(0, 0, 2), (1, 0, 4)]
    for clock, want in ((1.0, (1, 4, 11)), (2.0, (1, 11, 18)), (3.0, (1, 18, 20))):
        out = step(s, clock)
        assert out.phase is MIXED and ranges(out) == [want]
        assert [st.request.request_idx for st in out.decode_requests] == [0]
        assert out.num_scheduled_tokens == 1 + want[2] - want[1] <= 8
    last = step(s, 4.0)
    assert last.phase is DECODE and [st.request.request_idx for st in last.decode_requests] == [0, 1]
    assert last.prefill_chunks == ()


def test_mixed_update_takes_decode_tokens_first():
    s = scheduler(8, 4, mixed=True)
    a, b = states_with([2, 3], max_new=5)
    s.add_requests([a])
    step(s, 0.0)
    s.add_requests([b])
    out = s.schedule(1.0)
    assert out.phase is MIXED and out.decode_requests == (a,) and ranges(out) == [(1, 0, 3)]
    s.update_from_output(out, [11, 22], 1.0, stop_on_eos=False)
    assert a.generated == [7, 11] and b.generated == [22] and a.cache_length == 3 and b.cache_length == 3
    with pytest.raises(ValueError):
        s.update_from_output(s.schedule(2.0), [1], 2.0)


def test_mixed_chunk_cap_bounds_mixed_steps_only():
    """``mixed_chunk_tokens``: a MIXED step carries at most that many prompt tokens; a PREFILL step
    (nothing decoding) keeps the whole budget."""
    s = scheduler(16, 4, mixed=True, mixed_chunk_tokens=4)
    s.add_requests(states_with([2, 20], max_new=10))
    first = step(s, 0.0)
    assert first.phase is PREFILL and ranges(first) == [(0, 0, 2), (1, 0, 8)]
    for clock, want in ((1.0, (1, 8, 12)), (2.0, (1, 12, 16)), (3.0, (1, 16, 20))):
        out = step(s, clock)
        assert out.phase is MIXED and ranges(out) == [want] and out.num_scheduled_tokens == 5
    assert step(s, 4.0).phase is DECODE
    uncapped = scheduler(16, 4, mixed=True)
    uncapped.add_requests(states_with([2, 20], max_new=10))
    step(uncapped, 0.0)
    assert ranges(step(uncapped, 1.0)) == [(1, 8, 20)]
    for kwargs in ({"mixed": False, "mixed_chunk_tokens": 8}, {"mixed": True, "mixed_chunk_tokens": 3}):
        with pytest.raises(ValueError):
            scheduler(16, 4, **kwargs)


@pytest.mark.parametrize("budget,capacity", [(8, 2), (16, 4), (64, 8)])
def test_mixed_loop_generates_the_same_tokens(budget, capacity):
    lens, outs = [13, 4, 9, 2, 16, 30, 7], [5, 7, 3, 6, 4, 2, 9]
    arrivals = [0.0, 0.0, 3.0, 3.5, 20.0, 21.0, 200.0]
    requests = [Request(i, tuple(range(1, n + 1)), m, a) for i, (n, m, a) in enumerate(zip(lens, outs, arrivals))]
    plain = run_scheduler(FakeBackend(), requests, token_budget=budget, max_running_requests=capacity)
    backend = FakeBackend()
    mixed = run_scheduler(backend, requests, token_budget=budget, max_running_requests=capacity,
                          mixed_batching=True)
    assert mixed.tokens == plain.tokens
    assert any(e.phase is MIXED for e in mixed.events)
    assert all(e.num_scheduled_tokens <= budget for e in mixed.events if e.phase is not DECODE)
    # replay the executed steps: every request that has its first token and is not finished
    # decodes in every step (no decoder waits behind a prefill)
    decoding, made = set(), {}
    for kind, *rest in backend.executed:
        rows = rest[0] if kind != "prefill" else []
        chunks = rest[-1] if kind != "decode" else []
        assert set(rows) == decoding
        for i in rows:
            made[i] += 1
        for i, _, end in chunks:
            if end == lens[i]:
                made[i] = 1
                decoding.add(i)
        decoding -= {i for i in decoding if made[i] == outs[i]}
    assert max(len(e.request_ids) for e in mixed.events) <= capacity
    assert backend.kv_cache_manager.num_used_blocks == 0
    assert sorted(i for e in mixed.events for i in e.finished_request_ids) == list(range(7))
    # a chunk cap in mixed steps changes the steps, not the tokens
    capped = run_scheduler(FakeBackend(), requests, token_budget=budget, max_running_requests=capacity,
                           mixed_batching=True, mixed_chunk_tokens=capacity)
    assert capped.tokens == plain.tokens
    mixed_chunks = [sum(b - a for a, b in e.chunk_spans) for e in capped.events if e.phase is MIXED]
    assert mixed_chunks and max(mixed_chunks) <= capacity
    assert len(capped.events) >= len(mixed.events)


def test_percentile_is_nearest_rank():
    # reference src/mini_infra/utils.py:7-13: the ceil(n p / 100)-th smallest, at least the first
    assert percentile([], 50) == 0.0
    assert percentile([7.0], 95) == 7.0
    assert percentile(list(range(1, 11)), 50) == 5
    assert percentile(list(range(1, 11)), 95) == 10
    assert percentile(list(range(1, 11)), 1) == 1
    assert percentile([4.0, 1.0, 3.0, 2.0], 75) == 3.0


def test_latency_summary_from_the_logical_clock():
    """Fixed step costs make every timestamp known: one request arriving at 0 with a 6-token
    prompt (budget 8: one prefill step of 2.5 ms) and 3 output tokens (two decode steps of
    1.25 ms); a second request arriving at 100 ms, after the first finished."""
    requests = [Request(0, tuple(range(1, 7)), 3, 0.0), Request(1, tuple(range(1, 5)), 2, 100.0)]
    result = run_scheduler(FakeBackend(), requests, token_budget=8, max_running_requests=2)
    r0, r1 = result.requests
    assert (r0.queue_ms, r0.ttft_ms, r0.end_to_end_ms) == (0.0, 2.5, 5.0)
    assert r0.inter_token_latencies_ms == [1.25, 1.25]
    assert (r1.arrival_ms, r1.ttft_ms, r1.end_to_end_ms) == (100.0, 2.5, 3.75)
    summary = result.latency_summary()
    assert summary["ttft_ms_p50"] == 2.5 and summary["end_to_end_ms_p95"] == 5.0
    assert summary["itl_ms_p50"] == 1.25 and summary["itl_ms_max"] == 1.25
    assert result.busy_ms == 2.5 + 2 * 1.25 + 2.5 + 1.25
