"""PTO-WSP authoring API with an MI355X (gfx950) HIP backend.

The names exported here match the reference package ``pto_wsp``
(``python/pto_wsp/__init__.py:23-191``) for the data-parallel ``@kernel`` /
``@workload`` / ``P()`` path, so existing workloads move to the GPU by
changing only ``.compile(target="hip_gfx950")``.
"""

__version__ = "0.1.0"

from pto_wsp.types import Dense, DenseDyn, Ragged, Sparse, Symbol, Tensor, DType, Location
from pto_wsp.schedule import (
    DispatchPolicy,
    TimingPolicy,
    WindowMode,
    TaskWindow,
    DepsMode,
    Deps,
    ReadyPolicy,
    StartPolicy,
    TracePolicy,
    Pools,
    TaskGraphConfig,
)
from pto_wsp.program import Program, ProgramStats, TraceLevel, TraceEvent, ExecutionTrace, HIP_TARGETS
from pto_wsp.workload import Workload, Task
from pto_wsp.p_namespace import P, LoopVar, AffineIndex
from pto_wsp.kernel import pto, tl, Value, TileType, ScalarType, Tile, Scalar, KernelIR, OpKind
from pto_wsp.builder import (
    workload_decorator,
    kernel as kernel_decorator,
    Kernel,
    KernelRef,
    In,
    Out,
    InOut,
    Constexpr,
    KernelParam,
    extract_kernel_params,
    get_direction,
    get_inner_type,
)
from pto_wsp.errors import CompileError, ExecutionError, IRBridgeError, PtoError
from pto_wsp.primitives import (
    parallel_for,
    for_each,
    select,
    cond,
    task,
    combine,
    sequential,
    slot_set_u64,
    slot_load_u64,
)
from pto_wsp import scalar_expr
from pto_wsp.ptoisa_jit import ptoisa, ptoisa_kernel

workload = workload_decorator
kernel = kernel_decorator
jit_kernel = kernel

__all__ = [
    "Dense", "DenseDyn", "Ragged", "Sparse", "Symbol", "Tensor", "DType", "Location",
    "DispatchPolicy", "TimingPolicy", "WindowMode", "TaskWindow", "DepsMode", "Deps", "ReadyPolicy",
    "StartPolicy", "TracePolicy", "Pools", "TaskGraphConfig",
    "Program", "ProgramStats", "TraceLevel", "TraceEvent", "ExecutionTrace", "HIP_TARGETS",
    "Workload", "Task", "P", "LoopVar", "AffineIndex",
    "pto", "tl", "Value", "TileType", "ScalarType", "Tile", "Scalar", "KernelIR", "OpKind",
    "workload", "kernel", "jit_kernel", "ptoisa", "ptoisa_kernel", "Kernel", "KernelRef", "In", "Out", "InOut", "Constexpr",
    "KernelParam", "extract_kernel_params", "get_direction", "get_inner_type",
    "CompileError", "ExecutionError", "IRBridgeError", "PtoError",
    "parallel_for", "for_each", "select", "cond", "task", "combine", "sequential", "slot_set_u64", "slot_load_u64",
    "scalar_expr",
]
