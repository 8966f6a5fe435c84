"""Functional workload constructors (the reference's python/pto_wsp/primitives.py:14-189).

``parallel_for`` / ``for_each`` / ``select`` take a body callable of the loop
index, ``cond`` picks a branch by a ScalarExpr predicate at run time,
``combine`` / ``sequential`` group workloads, ``task`` is one kernel call, and
``slot_set_u64`` / ``slot_load_u64`` write the 256 u64 run-time slots that
predicates and schedule keys can read (``scalar_expr.slot_u64``).
"""

from __future__ import annotations

from typing import Any, Callable

from pto_wsp.workload import Workload

__all__ = ["parallel_for", "for_each", "select", "cond", "task", "combine", "sequential",
           "slot_set_u64", "slot_load_u64"]


def parallel_for(axis: Any, body: Callable[[Any], Any]) -> Workload:
    """Independent iterations over ``axis``; ``body(i)`` gives each iteration's workload."""
    return Workload("parallel_for", axis=axis, body=body)


def for_each(axis: Any, body: Callable[[Any], Any]) -> Workload:
    """Iterations over ``axis`` in order, each after the previous one."""
    return Workload("for_each", axis=axis, body=body)


def select(sparse: Any, body: Callable[[Any], Any]) -> Workload:
    """Iterations over the indices a ``Sparse`` axis selects at run time."""
    return Workload("select", sparse=sparse, body=body)


def cond(predicate: Any, then_workload: Any, else_workload: Any) -> Workload:
    """``then_workload`` when the ScalarExpr ``predicate`` is true at run time, else ``else_workload``."""
    return Workload("cond", predicate=predicate, then_workload=then_workload, else_workload=else_workload)


def _builder_add(w: Workload, needs_frame: bool) -> None:
    from pto_wsp.builder import get_current_builder

    b = get_current_builder()
    if b is not None and (b.frames or not needs_frame):
        b.add_child(w)


def task(kernel: Any, params: list, resources: Any) -> Workload:
    """One call of ``kernel`` with axis arguments ``params`` and ``resources`` = {param name: view}.

    Inside a ``@workload`` loop the task is also added to the enclosing loop.
    """
    if kernel is not None and hasattr(kernel, "trace") and hasattr(kernel, "name"):
        if not isinstance(resources, dict):
            raise TypeError("task(kernel=@kernel, ...) requires resources=dict[param_name -> Tensor/scalar]")
        w = Workload("task", kernel=kernel, params=params, resources=resources)
    else:
        w = Workload("task", kernel=str(kernel), params=params, resources=list(resources))
    _builder_add(w, needs_frame=True)
    return w


def combine(*workloads: Any) -> Workload:
    """Workloads with no order between them (the cycle model starts them together)."""
    return Workload("combine", workloads=list(workloads))


def sequential(*workloads: Any) -> Workload:
    """Workloads in order, each after the previous one completes."""
    return Workload("sequential", workloads=list(workloads))


def slot_set_u64(slot: int, value: int) -> Workload:
    """Set run-time slot ``slot`` to ``value`` (u64) when execution reaches this node."""
    w = Workload("slot_set_u64", slot=int(slot), value=int(value) & 0xFFFFFFFFFFFFFFFF)
    _builder_add(w, needs_frame=False)
    return w


def slot_load_u64(slot: int, tensor: Any, row: int = 0, col: int = 0) -> Workload:
    """Load element (row, col) of a tile view of ``tensor`` into run-time slot ``slot``.

    The view is indexed like a task's tile argument (its last two dimensions
    are the tile); the element is converted to u64 as C++ converts it.
    """
    w = Workload("slot_load_u64", slot=int(slot), tensor=tensor, row=int(row), col=int(col))
    _builder_add(w, needs_frame=False)
    return w
