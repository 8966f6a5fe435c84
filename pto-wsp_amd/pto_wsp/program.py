"""``Program``: a workload compiled for a target, plus execution statistics.

Mirrors ``python/pto_wsp/program.py`` of the reference (:194-751):

* ``Workload.compile(target)`` -> ``Program``; compile failures raise
  ``CompileError("Codegen compilation failed: ...")`` (:414-435);
* ``execute()`` is non-blocking and ``synchronize()`` waits (:670-743);
* ``stats.total_cycles`` is the analytic makespan of the cpu_sim cycle model
  and ``stats.task_count`` the number of tasks run;
* ``set_axis_sizes`` / ``set_symbol_u64|f32|ptr`` rebind DenseDyn extents and
  runtime symbols without recompiling (:348-381).

Targets: ``"hip_gfx950"`` (aliases ``"hip"``, ``"gfx950"``, ``"mi355x"``)
lowers the workload onto HIP kernels for one MI355X GPU.  Any other target
string is refused the way the reference's ``compile_codegen`` refuses an
unknown one (``src/python/pto_codegen.cpp:3433``).

Extensions over the reference: ``synchronize()`` raises ``ExecutionError``
when the device run failed, and ``stats`` also reports device time and the
host<->device staging time.
"""

from __future__ import annotations

import struct
import threading
import time
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Callable

from pto_wsp.errors import CompileError, ExecutionError

HIP_TARGETS = ("hip_gfx950", "hip", "gfx950", "mi355x")
_U64_MAX = (1 << 64) - 1


class TraceLevel(Enum):
    NONE = 0
    SUMMARY = 1
    TIMING = 2
    FULL = 3


@dataclass
class TraceEvent:
    name: str
    start_ms: float
    end_ms: float
    kind: str = "kernel"


@dataclass
class ExecutionTrace:
    events: list = field(default_factory=list)

    def add_event(self, ev: TraceEvent) -> None:
        self.events.append(ev)

    def to_chrome_trace(self) -> dict:
        return {"traceEvents": [
            {"name": e.name, "ph": "X", "ts": e.start_ms * 1000.0, "dur": (e.end_ms - e.start_ms) * 1000.0,
             "pid": 0, "tid": 0, "cat": e.kind} for e in self.events]}

    def print_summary(self) -> None:
        for e in self.events:
            print(f"{e.name}: {e.end_ms - e.start_ms:.4f} ms")


@dataclass
class ProgramStats:
    compile_time_ms: float = 0.0
    execute_time_ms: float = 0.0
    task_count: int = 0
    parallel_tasks: int = 0
    total_cycles: int = 0
    device_time_ms: float = 0.0
    h2d_ms: float = 0.0
    d2h_ms: float = 0.0
    launches: int = 0


class Program:
    def __init__(self, workload: Any, target: str, options: dict) -> None:
        self.workload = workload
        self.target = target
        self.options = dict(options or {})
        self.stats = ProgramStats()
        self.trace = ExecutionTrace()
        self._lock = threading.Lock()
        self._started = False
        self._pending = False
        self._trace_level = TraceLevel.NONE
        self._axis_sizes: dict[str, int] = self._infer_axis_sizes(workload)
        for k, v in (self.options.get("axis_sizes") or {}).items():
            self._axis_sizes[str(k)] = int(v)
        self._symbols_u64: dict[int, int] = {}
        self._symbols_ptr: dict[int, Any] = {}
        self._native = None
        self._codegen_tensors: list = []
        self._module_text = ""
        start = time.perf_counter()
        self._compile()
        self.stats.compile_time_ms = (time.perf_counter() - start) * 1000.0

    # -- properties -------------------------------------------------------
    @property
    def using_cpp_backend(self) -> bool:
        return self._native is not None

    @property
    def codegen_artifact_dir(self):
        return None

    @property
    def module_text(self) -> str:
        """The serialized codegen module this program was built from."""
        return self._module_text

    # -- tracing ----------------------------------------------------------
    def enable_tracing(self, level: TraceLevel = TraceLevel.TIMING) -> "Program":
        self._trace_level = level
        return self

    def disable_tracing(self) -> "Program":
        self._trace_level = TraceLevel.NONE
        return self

    def clear_trace(self) -> None:
        self.trace = ExecutionTrace()

    def register_kernel(self, name: str, impl: Callable, *, pass_task: bool = False) -> None:
        raise RuntimeError("program.register_kernel() is not supported in codegen-first mode")

    # -- runtime bindings ------------------------------------------------------
    def set_axis_sizes(self, axis_sizes: dict) -> None:
        for k, v in axis_sizes.items():
            self._axis_sizes[str(k)] = int(v)

    @staticmethod
    def _fnv1a_64(s: str) -> int:
        from pto_wsp.ir_bridge import fnv1a_64

        return fnv1a_64(s)

    def set_symbol_u64(self, name: str, value: int) -> None:
        self._symbols_u64[self._fnv1a_64(str(name))] = int(value) & 0xFFFFFFFFFFFFFFFF

    def set_symbol_f32(self, name: str, value: float) -> None:
        self.set_symbol_u64(name, struct.unpack("<I", struct.pack("<f", float(value)))[0])

    def set_symbol_ptr(self, name: str, arr: Any) -> None:
        self._symbols_ptr[self._fnv1a_64(str(name))] = arr

    @staticmethod
    def _infer_axis_sizes(workload: Any) -> dict:
        from pto_wsp.workload import Workload

        out: dict[str, int] = {}

        def walk(node: Any) -> None:
            if not isinstance(node, Workload):
                return
            kw = node._kwargs
            if node._kind in ("parallel_for", "for_each"):
                axis, var = kw.get("axis"), kw.get("var_name")
                if var and hasattr(axis, "size") and getattr(axis, "extent_view", None) is None:
                    try:
                        out[str(var)] = int(axis.size)
                    except Exception:  # noqa: BLE001
                        pass
                walk(kw.get("body"))
            elif node._kind in ("combine", "sequential"):
                for c in kw.get("workloads", []) or []:
                    walk(c)

        walk(workload)
        return out

    # -- compile ----------------------------------------------------------------
    def _compile(self) -> None:
        try:
            if self.target not in HIP_TARGETS:
                raise RuntimeError(f"compile_codegen: unsupported target: {self.target}")
            from pto_wsp import _hip
            from pto_wsp.ir_bridge import workload_to_codegen_ir

            name = self.workload._name if getattr(self.workload, "_name", None) else "main"
            build = workload_to_codegen_ir(self.workload, module_name=name)
            self._module_text = build.module
            self._codegen_tensors = build.tensors
            self._native = _hip.NativeProgram(build.module)
        except Exception as e:  # noqa: BLE001
            raise CompileError(f"Codegen compilation failed: {e}") from e

    # -- execution ----------------------------------------------------------
    def execute(self) -> None:
        """Enqueue the workload on the current HIP stream (non-blocking)."""
        with self._lock:
            if self._pending:
                raise RuntimeError("Program already started")
            self._started = True
            self._pending = True
        start = time.perf_counter()
        try:
            if self._native is None:
                raise RuntimeError("Program not compiled (missing native program)")
            res = self._native.launch(self._codegen_tensors, self._axis_sizes,
                                      self._symbols_u64, self._symbols_ptr)
        except Exception:
            with self._lock:
                self._pending = False
            raise
        # UINT64_MAX: the cycle model needs extent tensors that live on the
        # device; it runs at synchronize() (the reference also sets
        # total_cycles only when the run completes).
        self._cycles_pending = res.total_cycles == _U64_MAX
        if not self._cycles_pending:
            self.stats.total_cycles = int(res.total_cycles)
            self.stats.task_count = int(res.task_count)
        self.stats.launches = int(res.launches)
        self.stats.execute_time_ms = (time.perf_counter() - start) * 1000.0

    def synchronize(self) -> None:
        """Wait for the last ``execute()``; raises ``ExecutionError`` on device failure."""
        with self._lock:
            pending = self._pending
        if not pending:
            return
        try:
            timing = self._native.synchronize()
        except RuntimeError as e:
            raise ExecutionError(str(e)) from e
        finally:
            with self._lock:
                self._pending = False
        if getattr(self, "_cycles_pending", False):
            res = self._native.run_result()
            self.stats.total_cycles = int(res.total_cycles)
            self.stats.task_count = int(res.task_count)
            self._cycles_pending = False
        self.stats.device_time_ms = timing.device_ms
        self.stats.h2d_ms = timing.h2d_ms
        self.stats.d2h_ms = timing.d2h_ms
        if self._trace_level != TraceLevel.NONE:
            self.trace.add_event(TraceEvent("device", 0.0, timing.device_ms))

    def is_complete(self) -> bool:
        with self._lock:
            return not self._pending
