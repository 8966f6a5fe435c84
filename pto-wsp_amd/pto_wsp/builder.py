"""``@workload`` stack builder and the ``@kernel`` decorator.

Mirrors the reference builder (``python/pto_wsp/builder.py``):

* ``@workload`` runs the decorated body under a ``WorkloadBuilder``; ``P()``
  loops push frames and kernel calls append ``Workload("task", ...)`` leaves
  (builder.py:126-314).  Several top-level statements become a ``combine``.
* ``Kernel.trace()`` builds a ``KernelIR`` with parameters numbered first
  (builder.py:384-429); ``kernel[axes](**views)`` creates a task node whose
  ``params`` are the axis bindings and ``resources`` map parameter names to
  tensor views or scalars (builder.py:560-594).
* ``In/Out/InOut/Constexpr[...]`` carry ``_direction`` and ``_inner_type``
  (builder.py:675-787).
"""

from __future__ import annotations

import functools
import inspect
from contextvars import ContextVar
from dataclasses import dataclass, field
from typing import Any, Callable, Optional, get_type_hints

from pto_wsp.kernel import KernelIR, ScalarType, TileType, Value, ValueId, pto
from pto_wsp.types import DType, Tensor

_builder_stack: ContextVar[list] = ContextVar("pto_wsp_builder_stack", default=[])


@dataclass
class LoopFrame:
    kind: str
    axis: Any
    var_name: str
    children: list = field(default_factory=list)


@dataclass
class ConditionalFrame:
    predicate: Any
    then_body: list = field(default_factory=list)
    else_body: Optional[list] = None


@dataclass
class KernelParam:
    name: str
    direction: str
    inner_type: Any
    dtype: Any = None
    shape: Optional[tuple] = None


def _resolve_hints(func: Callable) -> dict:
    """``get_type_hints`` plus a fallback for string annotations that name
    objects visible only in the enclosing function (closure variables)."""
    if not getattr(func, "__annotations__", None):
        return {}
    try:
        return get_type_hints(func)
    except NameError:
        scope = dict(func.__globals__)
        if func.__closure__:
            for name, cell in zip(func.__code__.co_freevars, func.__closure__):
                try:
                    scope[name] = cell.cell_contents
                except ValueError:
                    pass
        return {k: (eval(v, scope) if isinstance(v, str) else v) for k, v in func.__annotations__.items()}


def extract_kernel_params(func: Callable) -> list[KernelParam]:
    """Parse ``In[Tile[...]]``-style annotations into ``KernelParam`` records."""
    hints = _resolve_hints(func)
    params: list[KernelParam] = []
    for name in inspect.signature(func).parameters:
        hint = hints.get(name)
        if hint is None:
            params.append(KernelParam(name, "in", None))
            continue
        direction = getattr(hint, "_direction", "in")
        inner = getattr(hint, "_inner_type", hint)
        dtype = shape = None
        if isinstance(inner, TileType):
            dtype, shape = inner.dtype, (inner.rows, inner.cols)
        elif isinstance(inner, ScalarType):
            dtype = inner.dtype
        params.append(KernelParam(name, direction, inner, dtype, shape))
    return params


class WorkloadBuilder:
    """Collects the loop frames and tasks produced while a ``@workload`` body runs."""

    def __init__(self, name: str, type_check: bool = True) -> None:
        self.name = name
        self.frames: list = []
        self.root_children: list = []
        self._pending_cond_workload = None
        self._var_counter = 0
        self._type_check = type_check
        self._type_errors: list[str] = []

    def push_frame(self, frame) -> None:
        self.frames.append(frame)

    def pop_frame(self):
        return self.frames.pop()

    def current_frame(self):
        return self.frames[-1] if self.frames else None

    def add_child(self, node: Any) -> None:
        if not self.frames:
            self.root_children.append(node)
            return
        frame = self.frames[-1]
        if isinstance(frame, LoopFrame):
            frame.children.append(node)
        elif frame.else_body is not None:
            frame.else_body.append(node)
        else:
            frame.then_body.append(node)

    def generate_var_name(self, prefix: str = "i") -> str:
        self._var_counter += 1
        return f"{prefix}_{self._var_counter}"

    # Builder-time checks: errors are collected (never raised here) and exposed
    # as ``Workload.type_errors``, like the reference's non-fail-fast checker.
    def check_kernel_call(self, kernel: "Kernel", axes: tuple, args: dict) -> None:
        if not self._type_check:
            return
        for p in kernel._kernel_params:
            if p.direction == "constexpr":
                continue
            if isinstance(p.inner_type, TileType) and p.name not in args:
                self._type_errors.append(f"{self.name}.{kernel.name}: missing tensor argument '{p.name}'")
            if isinstance(p.inner_type, TileType) and p.name in args:
                view = args[p.name]
                if isinstance(view, Tensor) and len(view.shape) == 0:
                    self._type_errors.append(f"{self.name}.{kernel.name}: argument '{p.name}' is a rank-0 view")

    def check_axis_bounds(self, axis: Any, index: Any) -> None:
        return None

    def check_tensor_access(self, tensor: Any, indices: tuple) -> None:
        if self._type_check and isinstance(tensor, Tensor) and len(indices) > len(tensor.shape) and tensor.shape:
            self._type_errors.append(
                f"{self.name}: {len(indices)} indices into a rank-{len(tensor.shape)} tensor view")

    def get_type_errors(self) -> list:
        return list(self._type_errors)

    def has_type_errors(self) -> bool:
        return bool(self._type_errors)

    def build(self):
        from pto_wsp.workload import Workload

        if not self.root_children:
            return Workload("empty")
        if len(self.root_children) == 1:
            return self.root_children[0]
        return Workload("combine", workloads=list(self.root_children))


def get_current_builder() -> Optional[WorkloadBuilder]:
    stack = _builder_stack.get()
    return stack[-1] if stack else None


def push_builder(builder: WorkloadBuilder) -> None:
    _builder_stack.set(_builder_stack.get() + [builder])


def pop_builder() -> Optional[WorkloadBuilder]:
    stack = _builder_stack.get()
    if not stack:
        return None
    _builder_stack.set(stack[:-1])
    return stack[-1]


def workload_decorator(func: Callable | None = None, *, type_check: bool = True,
                       fail_on_type_error: bool = False):
    """``@workload`` / ``@workload(type_check=..., fail_on_type_error=...)``."""

    def decorator(fn: Callable):
        @functools.wraps(fn)
        def wrapper(*args, **kwargs):
            builder = WorkloadBuilder(fn.__name__, type_check=type_check)
            push_builder(builder)
            try:
                fn(*args, **kwargs)
                errors = builder.get_type_errors()
                if errors and fail_on_type_error:
                    raise TypeError(f"Type errors in workload '{fn.__name__}':\n" + "\n".join(errors))
                result = builder.build()
                result._type_errors = errors
                return result
            finally:
                pop_builder()

        wrapper._workload_name = fn.__name__
        wrapper._type_check = type_check
        return wrapper

    return decorator(func) if func is not None else decorator


class Kernel:
    """A traced tile kernel usable inside workloads as ``kernel[axes](**views)``."""

    def __init__(self, func: Callable, **options) -> None:
        self.func = func
        self.name = func.__name__
        self.options = options
        self._signature = dict(getattr(func, "__annotations__", {}) or {})
        self._kernel_params = extract_kernel_params(func)
        functools.update_wrapper(self, func)

    @property
    def signature(self) -> dict:
        return self._signature

    def _trace(self, *args, **kwargs) -> KernelIR:
        ValueId.reset()
        ir = KernelIR(name=self.name, params=[])
        pto._current_ir = ir
        try:
            by_name = {p.name: p for p in self._kernel_params}
            values = {}
            for name in inspect.signature(self.func).parameters:
                meta = by_name.get(name)
                if meta is None or meta.inner_type is None:
                    val = Value.tile(32, 128, DType.F16, name=name)
                elif isinstance(meta.inner_type, TileType) and meta.shape is not None:
                    rows, cols = meta.shape
                    val = Value.tile(rows, cols, meta.dtype or DType.F16, meta.inner_type.location, name)
                elif isinstance(meta.inner_type, ScalarType):
                    val = Value.scalar(meta.dtype or DType.F32, name=name)
                else:
                    val = Value.scalar(DType.F32, name=name)
                values[name] = val
                ir.params.append((name, val))
            if self.options.get("cpp_src") is None and self.options.get("cpp_file_src") is None:
                self.func(**values)
        finally:
            pto._current_ir = None
        return ir

    def trace(self, **kwargs) -> KernelIR:
        return self._trace(**kwargs)

    def compile(self, target: str = "hip_gfx950", **kwargs):
        raise RuntimeError(
            "Kernel.compile() is not supported in codegen-first mode; "
            "compile the enclosing workload with workload.compile(target=...)")

    def _resources(self, args: tuple, kwargs: dict) -> dict:
        names = [n for n in inspect.signature(self.func).parameters if n != "return"]
        resources = {names[i]: a for i, a in enumerate(args) if i < len(names)}
        resources.update(kwargs)
        return resources

    def __call__(self, *args, **kwargs):
        builder = get_current_builder()
        if builder is None:
            return self._trace(*args, **kwargs)
        from pto_wsp.workload import Workload

        builder.check_kernel_call(self, (), kwargs)
        task = Workload("task", kernel=self, params=[], resources=self._resources(args, kwargs))
        builder.add_child(task)
        return task

    def __getitem__(self, axes) -> "_KernelCallWithAxes":
        return _KernelCallWithAxes(self, axes if isinstance(axes, tuple) else (axes,))


class _KernelCallWithAxes:
    def __init__(self, kernel: Kernel, axes: tuple) -> None:
        self.kernel = kernel
        self.kernel_ref = kernel
        self.axes = axes

    def __call__(self, *args, **kwargs):
        builder = get_current_builder()
        if builder is None:
            raise RuntimeError("Axis-bound kernel call must be inside @workload")
        from pto_wsp.workload import Workload

        builder.check_kernel_call(self.kernel, self.axes, kwargs)
        task = Workload("task", kernel=self.kernel, params=list(self.axes),
                        resources=self.kernel._resources(args, kwargs))
        builder.add_child(task)
        return task


def kernel(func: Callable | None = None, *, num_warps: int = 4, num_stages: int = 2,
           cpp_src: str | None = None, cpp_body_path: str | None = None,
           cpp_tu_path: str | None = None, cpp_includes: Optional[list] = None, **kwargs):
    """``@kernel`` decorator.

    ``cpp_src`` (or ``cpp_body_path``, a file holding one) gives the kernel a
    C++ body over the reference's task descriptor (``task->args``,
    ``task->tensor_ptrs``, ``task->tensor_strides``); the HIP backend compiles
    it as device code run by one thread per task.  ``cpp_tu_path`` names a
    whole translation unit that defines ``extern "C" uint64_t <kernel name>(
    const KernelTaskDesc*, CSPTContext*)`` against the reference's ABI headers
    (``pto/wsp/codegen/abi/kernel_abi.hpp``, ``ptoisa_bridge.hpp`` without the
    PTO-ISA tile API); the HIP backend compiles the file as device code and
    calls that function once per task.  ``cpp_includes`` (host include
    directories) is refused by that backend."""
    options = {"num_warps": num_warps, "num_stages": num_stages, **kwargs}
    chosen = [x for x in (cpp_src, cpp_body_path, cpp_tu_path) if x is not None]
    if len(chosen) > 1:
        raise ValueError("kernel(): use only one of cpp_src / cpp_body_path / cpp_tu_path")
    if cpp_src is not None:
        options["cpp_src"] = str(cpp_src)
    elif cpp_body_path is not None:
        with open(cpp_body_path, encoding="utf-8") as f:
            options["cpp_src"] = f.read()
    elif cpp_tu_path is not None:
        with open(cpp_tu_path, encoding="utf-8") as f:
            options["cpp_file_src"] = f.read()
    if cpp_includes is not None:
        options["cpp_includes"] = [str(x) for x in cpp_includes]

    def decorator(fn: Callable) -> Kernel:
        return Kernel(fn, **options)

    return decorator(func) if func is not None else decorator


KernelRef = Kernel


class _DirectionMeta(type):
    def __getitem__(cls, item):
        return type(f"{cls.__name__}[{item}]", (cls,), {"_inner_type": item, "_direction": cls.__name__.lower()})


class In(metaclass=_DirectionMeta):
    _inner_type = None
    _direction = "in"


class Out(metaclass=_DirectionMeta):
    _inner_type = None
    _direction = "out"


class InOut(metaclass=_DirectionMeta):
    _inner_type = None
    _direction = "inout"


class Constexpr(metaclass=_DirectionMeta):
    _inner_type = None
    _direction = "constexpr"


def get_direction(hint) -> str:
    if hasattr(hint, "_direction"):
        return hint._direction
    if isinstance(hint, str):
        for prefix, d in (("InOut[", "inout"), ("In[", "in"), ("Out[", "out"), ("Constexpr[", "constexpr")):
            if hint.startswith(prefix):
                return d
    return "unknown"


def get_inner_type(hint):
    return getattr(hint, "_inner_type", None)
