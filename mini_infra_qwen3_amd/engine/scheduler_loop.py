"""The continuous-batching loop and its summary metrics.

Loop semantics of the reference's ``_run_schedule_loop`` (src/mini_infra/engine/scheduler_loop.py:47-134):
a logical clock starts at the first arrival; each iteration moves arrived requests into the waiting
queue, asks the scheduler for a step, executes it and advances the clock by the step's
``model_ms + cache_ms``; an idle scheduler jumps the clock to the next arrival.  Summary metrics
follow ``summarize_schedule`` (src/mini_infra/engine/metrics.py:330-430): ``busy_ms`` is the sum of
step times and ``throughput_tok_s = output tokens * 1000 / busy_ms``.

``step_clock`` (not in the reference) replaces the measured step time on the logical clock by a
function of the plan, which makes the schedule independent of timing: two backends given the same
``step_clock`` execute identical step sequences.
"""

from __future__ import annotations

import gc
import math
import time
from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

from mini_infra_qwen3_amd.core.scheduler import (
    ArrivalQueue,
    IterationScheduler,
    RequestState,
    SchedulePhase,
    SchedulerOutput,
)
from mini_infra_qwen3_amd.core.types import Request
from mini_infra_qwen3_amd.device import synchronize


@dataclass(frozen=True)
class ScheduleEvent:
    """One executed step (reference metrics.py:269-289, the fields this path reports)."""

    phase: SchedulePhase
    request_ids: tuple[int, ...]
    admitted_request_ids: tuple[int, ...]
    finished_request_ids: tuple[int, ...]
    chunk_spans: tuple[tuple[int, int], ...]
    num_scheduled_tokens: int
    num_generated_tokens: int
    step_ms: float
    model_ms: float
    cache_ms: float
    live_kv_cache_bytes: int


def percentile(values: Sequence[float], percent: float) -> float:
    """Nearest-rank percentile, 0.0 for no values (reference src/mini_infra/utils.py:7-13): the
    ceil(n * percent / 100)-th smallest value, at least the first."""
    if not values:
        return 0.0
    ordered = sorted(values)
    rank = max(1, math.ceil(len(ordered) * percent / 100))
    return ordered[min(rank, len(ordered)) - 1]


@dataclass(frozen=True)
class RequestLatency:
    """Logical-clock timeline of one request (reference core/types.py:278-304), in ms."""

    request_idx: int
    arrival_ms: float
    admitted_ms: float
    first_token_ms: float
    completion_ms: float
    token_times_ms: tuple[float, ...]

    @property
    def queue_ms(self) -> float:
        return self.admitted_ms - self.arrival_ms

    @property
    def ttft_ms(self) -> float:
        return self.first_token_ms - self.arrival_ms

    @property
    def end_to_end_ms(self) -> float:
        return self.completion_ms - self.arrival_ms

    @property
    def inter_token_latencies_ms(self) -> list[float]:
        return [b - a for a, b in zip(self.token_times_ms, self.token_times_ms[1:])]


@dataclass(frozen=True)
class ScheduleResult:
    """Generated tokens per request (request_idx order), the step events and the summary."""

    tokens: dict[int, list[int]]
    events: list[ScheduleEvent]
    busy_ms: float
    model_ms: float
    cache_ms: float
    wall_ms: float
    makespan_ms: float
    num_output_tokens: int
    requests: tuple[RequestLatency, ...] = ()

    def latency_summary(self) -> dict[str, float]:
        """Queue, TTFT, end-to-end and inter-token latency percentiles over the requests, as the
        reference's schedule metrics report them (src/mini_infra/engine/metrics.py:370,426-434)."""
        itls = [x for r in self.requests for x in r.inter_token_latencies_ms]
        return {
            "queue_ms_p50": percentile([r.queue_ms for r in self.requests], 50),
            "queue_ms_p95": percentile([r.queue_ms for r in self.requests], 95),
            "ttft_ms_p50": percentile([r.ttft_ms for r in self.requests], 50),
            "ttft_ms_p95": percentile([r.ttft_ms for r in self.requests], 95),
            "end_to_end_ms_p50": percentile([r.end_to_end_ms for r in self.requests], 50),
            "end_to_end_ms_p95": percentile([r.end_to_end_ms for r in self.requests], 95),
            "itl_ms_p50": percentile(itls, 50),
            "itl_ms_p95": percentile(itls, 95),
            "itl_ms_max": max(itls, default=0.0),
        }

    @property
    def throughput_tok_s(self) -> float:
        return self.num_output_tokens * 1000.0 / self.busy_ms if self.busy_ms else 0.0

    @property
    def wall_tok_s(self) -> float:
        return self.num_output_tokens * 1000.0 / self.wall_ms if self.wall_ms else 0.0

    def phase_ms(self, phase: SchedulePhase) -> float:
        return sum(e.step_ms for e in self.events if e.phase is phase)

    def num_steps(self, phase: SchedulePhase) -> int:
        return sum(1 for e in self.events if e.phase is phase)


@torch.inference_mode()
def run_scheduler(backend, requests: Sequence[Request], token_budget: int = 2048,
                  max_running_requests: int | None = None, eos_token_id: int | None = None,
                  stop_on_eos: bool = True,
                  step_clock: Callable[[SchedulerOutput], float] | None = None,
                  mixed_batching: bool = False, mixed_chunk_tokens: int | None = None) -> ScheduleResult:
    """Runs ``requests`` to completion on ``backend`` (``execute_prefill`` / ``execute_decode`` and a
    ``kv_cache_manager``) with continuous batching and chunked prefill under ``token_budget``.

    ``max_running_requests`` defaults to the number of requests (reference scheduler_loop.py:162-163).
    ``mixed_batching`` runs decode rows and prefill chunks in the same step (``execute_mixed``), with
    at most ``mixed_chunk_tokens`` prompt tokens in such a step when given.

    While the loop runs, the objects that exist when it starts (model, pool, graphs) are frozen out
    of Python's cyclic garbage collector (``gc.freeze``, undone on return): a full collection over
    them took 36-64 ms, and one that fell inside a step's host enqueue added that much to the step.
    """
    if not requests:
        raise ValueError("requests must not be empty")
    if len({r.request_idx for r in requests}) != len(requests):
        raise ValueError("request_idx must be unique")
    mrr = max_running_requests if max_running_requests is not None else len(requests)
    states = [RequestState(r) for r in requests]
    arrivals = ArrivalQueue(states)
    clock_ms = min(r.arrival_ms for r in requests)
    scheduler = IterationScheduler(token_budget, mrr, backend.kv_cache_manager, mixed=mixed_batching,
                                   mixed_chunk_tokens=mixed_chunk_tokens)
    device = getattr(backend, "device", torch.device("cpu"))
    freeze = gc.isenabled()
    if freeze:
        gc.collect()
        gc.freeze()
    try:
        events, wall_ms = _loop(backend, scheduler, arrivals, clock_ms, device, step_clock, eos_token_id,
                                stop_on_eos)
    finally:
        if freeze:
            gc.unfreeze()
    return ScheduleResult(
        tokens={s.request.request_idx: list(s.generated) for s in sorted(states, key=lambda s: s.request.request_idx)},
        events=events,
        busy_ms=sum(e.step_ms for e in events),
        model_ms=sum(e.model_ms for e in events),
        cache_ms=sum(e.cache_ms for e in events),
        wall_ms=wall_ms,
        makespan_ms=max(s.completion_ms for s in states) - min(r.arrival_ms for r in requests),
        num_output_tokens=sum(len(s.generated) for s in states),
        requests=tuple(RequestLatency(s.request.request_idx, s.request.arrival_ms, s.admitted_ms, s.first_token_ms,
                                      s.completion_ms, tuple(s.token_times_ms))
                       for s in sorted(states, key=lambda s: s.request.request_idx)),
    )


def _loop(backend, scheduler: IterationScheduler, arrivals: ArrivalQueue, clock_ms: float, device: torch.device,
          step_clock: Callable[[SchedulerOutput], float] | None, eos_token_id: int | None,
          stop_on_eos: bool) -> tuple[list[ScheduleEvent], float]:
    """The loop of ``run_scheduler``: the step events and the wall time in ms."""
    events: list[ScheduleEvent] = []
    synchronize(device)
    wall_start = time.perf_counter()
    while len(arrivals) or scheduler.has_unfinished_requests:
        scheduler.add_requests(arrivals.pop_arrived(clock_ms))
        output = scheduler.schedule(clock_ms)
        if output is None:
            clock_ms = arrivals.next_arrival_ms()
            continue
        if output.phase is SchedulePhase.PREFILL:
            step = backend.execute_prefill(output.prefill_chunks)
        elif output.phase is SchedulePhase.MIXED:
            step = backend.execute_mixed(output.decode_requests, output.prefill_chunks)
        else:
            step = backend.execute_decode(output.scheduled_requests)
        step_ms = step.model_ms + step.cache_ms
        clock_ms += step_ms if step_clock is None else step_clock(output)
        finished = scheduler.update_from_output(output, step.next_tokens, clock_ms, eos_token_id, stop_on_eos)
        events.append(ScheduleEvent(
            phase=output.phase,
            request_ids=tuple(s.request.request_idx for s in output.scheduled_requests),
            admitted_request_ids=tuple(c.state.request.request_idx for c in output.prefill_chunks if c.start == 0),
            finished_request_ids=tuple(s.request.request_idx for s in finished),
            chunk_spans=tuple((c.start, c.end) for c in output.prefill_chunks),
            num_scheduled_tokens=output.num_scheduled_tokens,
            num_generated_tokens=len(step.next_tokens),
            step_ms=step_ms, model_ms=step.model_ms, cache_ms=step.cache_ms,
            live_kv_cache_bytes=step.live_kv_cache_bytes,
        ))
    synchronize(device)
    return events, (time.perf_counter() - wall_start) * 1000.0


__all__ = ["RequestLatency", "ScheduleEvent", "ScheduleResult", "percentile", "run_scheduler"]
