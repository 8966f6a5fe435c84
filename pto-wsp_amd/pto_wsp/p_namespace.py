"""``P`` loop constructors for ``@workload`` bodies.

Mirrors the reference (``python/pto_wsp/p_namespace.py``):

* ``P(a, b)`` / ``P.grid`` yields loop variables once and wraps the collected
  body in nested ``parallel_for`` nodes, outermost axis first (:49-115).
  Default variable names cycle through ``b h s d i j k l m n`` using the
  builder's counter (:230-254), so ``for x in P(batch)`` binds the runtime
  axis-size key ``"b"``.
* ``P.seq(axis, name="i")`` wraps its body in ``for_each`` (:118-161).
* ``P.sel`` / ``P.when`` / ``P.otherwise`` build ``select`` / ``cond`` nodes (:164-387).

Extension: loop variables support ``+``, ``-`` and ``*`` by integers, giving
``AffineIndex`` expressions ``c0 + sum(coef * var)`` usable as tensor indices
and as the extent of ``DenseDyn`` bound tensors.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Optional

from pto_wsp.builder import ConditionalFrame, LoopFrame, get_current_builder


class AffineIndex:
    """``const + sum(coef * var)`` over loop variables (integer coefficients)."""

    def __init__(self, terms: dict[str, int] | None = None, const: int = 0) -> None:
        self.terms = {k: int(v) for k, v in (terms or {}).items() if int(v) != 0}
        self.const = int(const)

    @staticmethod
    def of(x: Any) -> "AffineIndex":
        if isinstance(x, AffineIndex):
            return x
        if isinstance(x, LoopVar):
            return AffineIndex({x.name: 1}, 0)
        if isinstance(x, int):
            return AffineIndex({}, x)
        raise TypeError(f"not an affine index operand: {x!r}")

    def __add__(self, other: Any) -> "AffineIndex":
        o = AffineIndex.of(other)
        terms = dict(self.terms)
        for k, v in o.terms.items():
            terms[k] = terms.get(k, 0) + v
        return AffineIndex(terms, self.const + o.const)

    __radd__ = __add__

    def __sub__(self, other: Any) -> "AffineIndex":
        return self + AffineIndex.of(other) * -1

    def __rsub__(self, other: Any) -> "AffineIndex":
        return AffineIndex.of(other) + self * -1

    def __mul__(self, k: Any) -> "AffineIndex":
        if not isinstance(k, int):
            raise TypeError("affine indices multiply by integers only")
        return AffineIndex({n: c * k for n, c in self.terms.items()}, self.const * k)

    __rmul__ = __mul__

    def __repr__(self) -> str:
        parts = [f"{c}*{n}" for n, c in self.terms.items()]
        return " + ".join(parts + [str(self.const)])


class LoopVar:
    """Symbolic loop variable; ``name`` is its key in the generated loop nest."""

    def __init__(self, name: str, axis: Any, index: int = 0) -> None:
        self.name = name
        self.axis = axis
        self.index = index

    def __hash__(self) -> int:
        return hash(self.name)

    def __eq__(self, other: Any) -> bool:
        return isinstance(other, LoopVar) and other.name == self.name and other.axis is self.axis

    def __repr__(self) -> str:
        return f"LoopVar({self.name})"

    def __add__(self, other: Any) -> AffineIndex:
        return AffineIndex.of(self) + other

    __radd__ = __add__

    def __sub__(self, other: Any) -> AffineIndex:
        return AffineIndex.of(self) - other

    def __rsub__(self, other: Any) -> AffineIndex:
        return AffineIndex.of(other) - AffineIndex.of(self)

    def __mul__(self, k: Any) -> AffineIndex:
        return AffineIndex.of(self) * k

    __rmul__ = __mul__


def _body_of(children: list, multi_kind: str):
    from pto_wsp.workload import Workload

    if not children:
        return Workload("empty")
    if len(children) == 1:
        return children[0]
    return Workload(multi_kind, workloads=list(children))


def _require_builder(what: str):
    builder = get_current_builder()
    if builder is None:
        raise RuntimeError(f"{what} used outside @workload context")
    return builder


class ParallelGridIterator:
    def __init__(self, axes: tuple, var_names: list[str]) -> None:
        self.axes = axes
        self.var_names = var_names

    def __iter__(self):
        from pto_wsp.workload import Workload

        builder = _require_builder("P()")
        loop_vars = [LoopVar(n, a) for n, a in zip(self.var_names, self.axes)]
        frame = LoopFrame(kind="parallel", axis=self.axes, var_name=",".join(self.var_names))
        builder.push_frame(frame)
        yield loop_vars[0] if len(loop_vars) == 1 else tuple(loop_vars)
        builder.pop_frame()
        node = _body_of(frame.children, "combine")
        for axis, var in zip(reversed(self.axes), reversed(loop_vars)):
            node = Workload("parallel_for", axis=axis, body=node, var_name=var.name)
        builder.add_child(node)


class SequentialIterator:
    def __init__(self, axis: Any, var_name: str) -> None:
        self.axis = axis
        self.var_name = var_name

    def __iter__(self):
        from pto_wsp.workload import Workload

        builder = _require_builder("P.seq()")
        var = LoopVar(self.var_name, self.axis)
        frame = LoopFrame(kind="sequential", axis=self.axis, var_name=self.var_name)
        builder.push_frame(frame)
        yield var
        builder.pop_frame()
        body = _body_of(frame.children, "sequential")
        builder.add_child(Workload("for_each", axis=self.axis, body=body, var_name=self.var_name))


class SelectIterator:
    def __init__(self, sparse: Any, var_name: str) -> None:
        self.sparse = sparse
        self.var_name = var_name

    def __iter__(self):
        from pto_wsp.workload import Workload

        builder = _require_builder("P.sel()")
        var = LoopVar(self.var_name, self.sparse)
        frame = LoopFrame(kind="select", axis=self.sparse, var_name=self.var_name)
        builder.push_frame(frame)
        yield var
        builder.pop_frame()
        body = _body_of(frame.children, "combine")
        builder.add_child(Workload("select", sparse=self.sparse, body=body, var_name=self.var_name))


class PNamespace:
    _DEFAULT_NAMES = ["b", "h", "s", "d", "i", "j", "k", "l", "m", "n"]

    def __call__(self, *axes, **kwargs) -> ParallelGridIterator:
        return self.grid(*axes, **kwargs)

    def grid(self, *axes, names: Optional[list] = None) -> ParallelGridIterator:
        builder = _require_builder("P.grid()")
        if names is None:
            names = []
            for _ in axes:
                names.append(self._DEFAULT_NAMES[builder._var_counter % len(self._DEFAULT_NAMES)])
                builder._var_counter += 1
        return ParallelGridIterator(axes, list(names))

    def seq(self, axis: Any, name: str = "i") -> SequentialIterator:
        return SequentialIterator(axis, name)

    def sel(self, sparse: Any, name: str = "e") -> SelectIterator:
        return SelectIterator(sparse, name)

    @contextmanager
    def when(self, predicate: Any):
        from pto_wsp.workload import Workload

        builder = _require_builder("P.when()")
        frame = ConditionalFrame(predicate=predicate)
        builder.push_frame(frame)
        try:
            yield
        finally:
            builder.pop_frame()
            node = Workload("cond", predicate=predicate,
                            then_workload=_body_of(frame.then_body, "combine"),
                            else_workload=Workload("empty"))
            builder.add_child(node)
            builder._pending_cond_workload = node

    @contextmanager
    def otherwise(self):
        builder = _require_builder("P.otherwise()")
        pending = builder._pending_cond_workload
        if pending is None or pending._kind != "cond":
            raise RuntimeError("P.otherwise() must follow P.when()")
        frame = ConditionalFrame(predicate=None, then_body=[], else_body=[])
        builder.push_frame(frame)
        try:
            yield
        finally:
            builder.pop_frame()
            pending._kwargs["else_workload"] = _body_of(frame.else_body or [], "combine")
            builder._pending_cond_workload = None


P = PNamespace()
