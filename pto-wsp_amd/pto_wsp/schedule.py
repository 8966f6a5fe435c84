"""Schedule policy objects (``python/pto_wsp/schedule.py`` in the reference).

Only ``DispatchPolicy`` (lane count; round-robin assignment, or a lane of
``key % lanes`` for ``affinity`` / ``hash`` / ``dispatch_by``, whose key
function is traced into a ScalarExpr over ``t.params``, ``t.tags`` and
``t.get(axis)``) and a ``TaskWindow`` in units of tasks with ``STALL``
overflow change anything: they feed the analytic cycle model that
``Program.stats.total_cycles`` reports (``src/python/pto_codegen.cpp:1527-1607,
2679-2690``).  The rest are accepted and carried.
"""

from __future__ import annotations

from enum import Enum
from typing import Any, Callable


class WindowMode(Enum):
    STALL = "stall"
    ABORT = "abort"
    BENCHMARK = "benchmark"


class DispatchPolicy:
    def __init__(self, kind: str, **kwargs) -> None:
        self._kind = kind
        self._kwargs = kwargs

    @staticmethod
    def round_robin(num_aicpus: int) -> "DispatchPolicy":
        return DispatchPolicy("round_robin", num_aicpus=num_aicpus)

    @staticmethod
    def affinity(key_fn: Callable[[Any], Any], num_aicpus: int = 0) -> "DispatchPolicy":
        return DispatchPolicy("affinity", key_fn=key_fn, num_aicpus=num_aicpus)

    @staticmethod
    def hash(key_fn: Callable[[Any], Any], num_aicpus: int = 0) -> "DispatchPolicy":
        return DispatchPolicy("hash", key_fn=key_fn, num_aicpus=num_aicpus)

    @staticmethod
    def work_steal() -> "DispatchPolicy":
        return DispatchPolicy("work_steal")

    @staticmethod
    def dispatch_by(fn: Callable[[Any], int], num_aicpus: int = 0) -> "DispatchPolicy":
        return DispatchPolicy("dispatch_by", fn=fn, num_aicpus=num_aicpus)

    def __repr__(self) -> str:
        return f"DispatchPolicy.{self._kind}({self._kwargs})"


class TimingPolicy:
    def __init__(self, kind: str, **kwargs) -> None:
        self._kind = kind
        self._kwargs = kwargs

    @staticmethod
    def batched(n: int) -> "TimingPolicy":
        return TimingPolicy("batched", n=n)

    @staticmethod
    def interleaved(streams: int) -> "TimingPolicy":
        return TimingPolicy("interleaved", streams=streams)

    @staticmethod
    def rate_limit(tasks_per_ms: int) -> "TimingPolicy":
        return TimingPolicy("rate_limit", tasks_per_ms=tasks_per_ms)


TimingPolicy.immediate = TimingPolicy("immediate")


class TaskWindow:
    def __init__(self, size: int, unit: str = "tasks", mode: WindowMode = WindowMode.STALL) -> None:
        if unit not in ("tasks", "bytes", "entries"):
            raise ValueError(f"Invalid unit: {unit}")
        self.size = int(size)
        self.unit = unit
        self.mode = mode


class DepsMode(Enum):
    INFER_TENSOR_MAP_EXACT = "infer_tensor_map_exact"
    INFER_BYTES_OVERLAP = "infer_bytes_overlap"
    EXPLICIT = "explicit"
    HYBRID = "hybrid"


class _Policy:
    def __init__(self, kind: str, **kwargs) -> None:
        self._kind = kind
        self._kwargs = kwargs

    def __repr__(self) -> str:
        return f"{type(self).__name__}.{self._kind}"


class Deps(_Policy):
    @staticmethod
    def infer_tensor_map_exact() -> "Deps":
        return Deps(DepsMode.INFER_TENSOR_MAP_EXACT.value)

    @staticmethod
    def infer_bytes_overlap() -> "Deps":
        return Deps(DepsMode.INFER_BYTES_OVERLAP.value)

    @staticmethod
    def explicit() -> "Deps":
        return Deps(DepsMode.EXPLICIT.value)

    @staticmethod
    def hybrid() -> "Deps":
        return Deps(DepsMode.HYBRID.value)


class ReadyPolicy(_Policy):
    @staticmethod
    def fifo() -> "ReadyPolicy":
        return ReadyPolicy("fifo")

    @staticmethod
    def work_steal() -> "ReadyPolicy":
        return ReadyPolicy("work_steal")

    @staticmethod
    def fair() -> "ReadyPolicy":
        return ReadyPolicy("fair")

    @staticmethod
    def priority(priority_fn: Callable[[Any], int]) -> "ReadyPolicy":
        return ReadyPolicy("priority", priority_fn=priority_fn)


class StartPolicy(_Policy):
    @staticmethod
    def threshold(n: int) -> "StartPolicy":
        return StartPolicy("threshold", n=n)

    @staticmethod
    def after_orchestration() -> "StartPolicy":
        return StartPolicy("after_orchestration")


class TracePolicy(_Policy):
    @staticmethod
    def none() -> "TracePolicy":
        return TracePolicy("none")

    @staticmethod
    def cycles(cost_fn: Callable | None = None) -> "TracePolicy":
        return TracePolicy("cycles", cost_fn=cost_fn)


class Pools(_Policy):
    @staticmethod
    def single() -> "Pools":
        return Pools("single")

    @staticmethod
    def by_exec_unit() -> "Pools":
        return Pools("by_exec_unit")

    @staticmethod
    def custom(pool_fn: Callable[[Any], str]) -> "Pools":
        return Pools("custom", pool_fn=pool_fn)


class TaskGraphConfig:
    def __init__(self, deps: Deps | None = None, window: TaskWindow | None = None,
                 pools: Pools | None = None, ready: ReadyPolicy | None = None,
                 start: StartPolicy | None = None, trace: TracePolicy | None = None) -> None:
        self.deps = deps or Deps.infer_tensor_map_exact()
        self.window = window or TaskWindow(8192, "tasks", WindowMode.STALL)
        self.pools = pools or Pools.single()
        self.ready = ready or ReadyPolicy.fifo()
        self.start = start or StartPolicy.after_orchestration()
        self.trace = trace or TracePolicy.none()
