"""``Workload`` tree node and its combinator-style schedule API.

Mirrors ``python/pto_wsp/workload.py`` of the reference: every schedule call
returns a shallow copy (:619-642); ``compile(target)`` builds a ``Program``
(:597-608); ``task_graph`` attaches a ``TaskGraphConfig`` and clears the
stream settings (:526-595).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable, Optional


@dataclass
class Schedule:
    dispatch: Any = None
    streams: int = 1
    stream_by: Optional[Callable] = None
    timing: Any = None

    def to_dict(self) -> dict:
        out: dict = {}
        if self.dispatch is not None:
            out["dispatch"] = self.dispatch
        if self.streams != 1:
            out["streams"] = self.streams
        if self.stream_by is not None:
            out["stream_by"] = self.stream_by
        if self.timing is not None:
            out["timing"] = self.timing
        return out


@dataclass
class Task:
    kernel: str
    params: list
    resources: list
    id: int = 0
    bindings: dict = field(default_factory=dict)

    def get(self, axis: str, default: int = 0) -> int:
        return self.bindings.get(axis, default)

    def get_axis_value(self, index: int) -> int:
        return self.params[index] if 0 <= index < len(self.params) else 0


def axis_extent(axis: Any) -> int:
    if isinstance(axis, int):
        return axis
    if hasattr(axis, "size"):
        return int(axis.size)
    if hasattr(axis, "__len__"):
        return len(axis)
    return 0


class Workload:
    """A node of the workload tree: ``task``, ``parallel_for``, ``for_each``,
    ``combine``, ``sequential``, ``select``, ``cond`` or ``empty``."""

    def __init__(self, kind: str, name: Optional[str] = None, **kwargs) -> None:
        self._kind = kind
        self._kwargs = kwargs
        self._name = name
        self._params: list = []
        self._schedule = Schedule()
        self._dispatch_policy = None
        self._stream_count = 1
        self._stream_by_fn = None
        self._timing_policy = None
        self._spatial_grid = None
        self._layouts: list = []
        self._task_graph_config = None
        self._type_errors: list = []

    def __repr__(self) -> str:
        return f"Workload({self._kind})"

    # -- enumeration (debugging aid; program order, loop vars bound) --------
    def enumerate(self) -> list[Task]:
        tasks: list[Task] = []
        self._enumerate(tasks, {})
        for i, t in enumerate(tasks):
            t.id = i
        return tasks

    def _enumerate(self, out: list, bindings: dict) -> None:
        kind = self._kind
        kw = self._kwargs
        if kind == "task":
            kernel = kw.get("kernel")
            name = getattr(kernel, "name", str(kernel))
            params = [bindings.get(p.name, 0) if hasattr(p, "name") else p for p in kw.get("params", [])]
            out.append(Task(name, params, list(kw.get("resources", {}).values()), 0, dict(bindings)))
        elif kind in ("parallel_for", "for_each"):
            body = kw.get("body")
            for i in range(axis_extent(kw.get("axis"))):
                if isinstance(body, Workload):
                    body._enumerate(out, {**bindings, kw.get("var_name", "i"): i})
        elif kind in ("combine", "sequential"):
            for w in kw.get("workloads", []) or []:
                w._enumerate(out, bindings)
        elif kind == "select":
            sparse = kw.get("sparse")
            body = kw.get("body")
            for idx in getattr(sparse, "indices", []):
                body._enumerate(out, {**bindings, kw.get("var_name", "e"): idx})
        elif kind == "cond":
            then_w = kw.get("then_workload")
            if isinstance(then_w, Workload):
                then_w._enumerate(out, bindings)

    # -- metadata -----------------------------------------------------------
    def named(self, name: str) -> "Workload":
        w = self._copy()
        w._name = name
        return w

    def with_params(self, *params) -> "Workload":
        w = self._copy()
        w._params = list(params)
        return w

    # -- schedule combinators ----------------------------------------------
    def dispatch(self, policy: Any) -> "Workload":
        w = self._copy()
        w._dispatch_policy = policy
        w._schedule.dispatch = policy
        return w

    def streams(self, count: int) -> "Workload":
        w = self._copy()
        w._stream_count = count
        w._schedule.streams = count
        return w

    def stream_by(self, key_fn: Callable) -> "Workload":
        w = self._copy()
        w._stream_by_fn = key_fn
        w._schedule.stream_by = key_fn
        return w

    def timing(self, policy: Any) -> "Workload":
        w = self._copy()
        w._timing_policy = policy
        w._schedule.timing = policy
        return w

    def spatial_map(self, grid: tuple) -> "Workload":
        w = self._copy()
        w._spatial_grid = grid
        return w

    def task_graph(self, deps: Any = None, window: Any = None, pools: Any = None,
                   ready: Any = None, start: Any = None, trace: Any = None) -> "Workload":
        from pto_wsp.schedule import TaskGraphConfig

        w = self._copy()
        w._task_graph_config = TaskGraphConfig(deps=deps, window=window, pools=pools,
                                               ready=ready, start=start, trace=trace)
        w._stream_count = None
        w._stream_by_fn = None
        return w

    def compile(self, target: str = "hip_gfx950", **options):
        from pto_wsp.program import Program

        return Program(self, target, options)

    @property
    def type_errors(self) -> list:
        return self._type_errors

    def has_type_errors(self) -> bool:
        return bool(self._type_errors)

    def _copy(self) -> "Workload":
        w = Workload(self._kind, name=self._name, **self._kwargs)
        w._params = list(self._params)
        w._schedule = Schedule(self._schedule.dispatch, self._schedule.streams,
                               self._schedule.stream_by, self._schedule.timing)
        w._dispatch_policy = self._dispatch_policy
        w._stream_count = self._stream_count
        w._stream_by_fn = self._stream_by_fn
        w._timing_policy = self._timing_policy
        w._spatial_grid = self._spatial_grid
        w._layouts = list(self._layouts)
        w._task_graph_config = self._task_graph_config
        w._type_errors = list(self._type_errors)
        return w
