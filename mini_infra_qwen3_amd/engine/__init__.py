"""Continuous-batching driver of the paged path: scheduler loop, paged backend, metrics."""

from mini_infra_qwen3_amd.engine.paged_backend import PagedScheduleBackend, ScheduleStepOutput
from mini_infra_qwen3_amd.engine.scheduler_loop import (RequestLatency, ScheduleEvent, ScheduleResult, percentile,
                                                        run_scheduler)

__all__ = ["PagedScheduleBackend", "RequestLatency", "ScheduleEvent", "ScheduleResult", "ScheduleStepOutput",
           "percentile", "run_scheduler"]
