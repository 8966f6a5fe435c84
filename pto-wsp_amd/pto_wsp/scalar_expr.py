"""Symbolic scalar expressions (ScalarExpr) for run-time predicates and schedule keys.

Mirrors the reference DSL (python/pto_wsp/scalar_expr.py): an immutable
expression tree with a C-like scalar type ("bool", "i64", "u64") built from
literals, loop variables (``axis``), u64 symbols, the 256 u64 run-time slots,
task parameters and task tags, combined with Python operators.  Nothing here
runs at execution time: the tree is serialized into the module text
(``to_text``) and evaluated by the native runtime with C++ operator semantics,
as the reference's emitted artifact does (src/python/pto_codegen.cpp:220-300).

Type rules (the same as the reference's):
* ``&`` / ``|`` are logical on bool operands and bitwise on u64 operands;
  ``^`` needs u64; ``~`` works on bool and u64; unary ``-`` on i64 and u64;
* ``<<`` / ``>>`` cast both sides to u64;
* comparisons give bool; arithmetic keeps the left operand's declared type;
* ``where(t, f)`` needs a bool predicate and branches of one type;
* Python's ``and`` / ``or`` / ``if`` cannot be overloaded and raise TypeError.
"""

from __future__ import annotations

from typing import Any, Callable

__all__ = [
    "Expr", "TaskExpr", "as_expr", "axis", "fnv1a_64", "slot_bool", "slot_i64", "slot_u64",
    "symbol_u64", "task_param", "trace_task_fn",
]

_MASK = 0xFFFFFFFFFFFFFFFF
_TYPES = ("bool", "i64", "u64")
_TYPE_CODE = {"bool": "b", "i64": "i", "u64": "u"}


def fnv1a_64(s: str) -> int:
    """FNV-1a 64-bit hash of the UTF-8 bytes of ``s`` (the id scheme of symbols and axes)."""
    h = 0xCBF29CE484222325
    for byte in str(s).encode("utf-8"):
        h = ((h ^ byte) * 0x100000001B3) & _MASK
    return h


class Expr:
    """One node of a scalar expression: ``kind``, declared ``type`` and up to three fields."""

    __slots__ = ("kind", "type", "a", "b", "c")

    def __init__(self, kind: str, type: str, a: Any = None, b: Any = None, c: Any = None):
        if type not in _TYPES:
            raise TypeError(f"Unknown scalar type: {type}")
        object.__setattr__(self, "kind", kind)
        object.__setattr__(self, "type", type)
        object.__setattr__(self, "a", a)
        object.__setattr__(self, "b", b)
        object.__setattr__(self, "c", c)

    def __setattr__(self, name, value):  # immutable, like a frozen dataclass
        raise AttributeError("Expr is immutable")

    def __hash__(self) -> int:
        return hash((self.kind, self.type, self.a, self.b, self.c))

    def __repr__(self) -> str:
        return f"Expr({self.to_debug_str()})"

    # -- rendering ------------------------------------------------------------
    def to_debug_str(self) -> str:
        k = self.kind
        if k.startswith("lit_"):
            return repr(self.a)
        if k == "task_param":
            return f"task.params[{self.a}]"
        if k == "kernel_scalar":
            return f"scalar[{self.a}]"
        if k == "axis_var":
            return f"axis({self.a:#x})"
        if k == "task_tag_u64":
            return f"tag({self.a:#x})"
        if k == "symbol_u64":
            return f"symbol({self.a:#x})"
        if k.startswith("slot_"):
            return f"{k}({self.a})"
        if k == "unary":
            return f"({self.a} {self.b.to_debug_str()})"
        if k == "binary":
            return f"({self.b.to_debug_str()} {self.a} {self.c.to_debug_str()})"
        if k == "ternary":
            return f"({self.a.to_debug_str()} ? {self.b.to_debug_str()} : {self.c.to_debug_str()})"
        if k == "cast":
            return f"({self.type})({self.a.to_debug_str()})"
        return f"<expr:{k}>"

    def to_text(self) -> str:
        """Prefix token form read by the native module parser and the oracle."""
        out: list[str] = []
        _emit(self, out)
        return " ".join(out)

    # -- Python truthiness is not an expression ------------------------------
    def __bool__(self) -> bool:
        raise TypeError("ScalarExpr cannot be used with Python 'and/or' or in 'if'. Use '&'/'|' or Expr.where().")

    def where(self, then_expr: Any, else_expr: Any) -> "Expr":
        if self.type != "bool":
            raise TypeError("where() requires a bool predicate Expr")
        t, f = as_expr(then_expr), as_expr(else_expr)
        if t.type != f.type:
            raise TypeError("where() branch type mismatch")
        return Expr("ternary", t.type, self, t, f)

    # -- unary -----------------------------------------------------------------
    def __invert__(self) -> "Expr":
        if self.type == "bool":
            return Expr("unary", "bool", "!", self)
        if self.type == "u64":
            return Expr("unary", "u64", "~", self)
        raise TypeError("~ supported for bool/u64 only")

    def __neg__(self) -> "Expr":
        if self.type == "bool":
            raise TypeError("Unary - supported for i64/u64 only")
        return Expr("unary", self.type, "-", self)

    # -- arithmetic (declared type: the left operand's) ------------------------
    def _arith(self, op: str, other: Any) -> "Expr":
        return Expr("binary", self.type, op, self, as_expr(other))

    def __add__(self, other: Any) -> "Expr":
        return self._arith("+", other)

    def __sub__(self, other: Any) -> "Expr":
        return self._arith("-", other)

    def __mul__(self, other: Any) -> "Expr":
        return self._arith("*", other)

    def __floordiv__(self, other: Any) -> "Expr":
        return self._arith("/", other)

    def __mod__(self, other: Any) -> "Expr":
        return self._arith("%", other)

    # -- logical / bitwise -----------------------------------------------------
    def _logic(self, other: Any, bool_op: str | None, u64_op: str, sym: str) -> "Expr":
        rhs = as_expr(other)
        if bool_op is not None and self.type == rhs.type == "bool":
            return Expr("binary", "bool", bool_op, self, rhs)
        if self.type == rhs.type == "u64":
            return Expr("binary", "u64", u64_op, self, rhs)
        if bool_op is None:
            raise TypeError(f"{sym} requires u64")
        raise TypeError(f"{sym} requires both bool or both u64")

    def __and__(self, other: Any) -> "Expr":
        return self._logic(other, "&&", "&", "&")

    def __or__(self, other: Any) -> "Expr":
        return self._logic(other, "||", "|", "|")

    def __xor__(self, other: Any) -> "Expr":
        return self._logic(other, None, "^", "^")

    def __lshift__(self, other: Any) -> "Expr":
        return Expr("binary", "u64", "<<", self.cast_u64(), as_expr(other).cast_u64())

    def __rshift__(self, other: Any) -> "Expr":
        return Expr("binary", "u64", ">>", self.cast_u64(), as_expr(other).cast_u64())

    # -- comparisons -----------------------------------------------------------
    def _cmp(self, op: str, other: Any) -> "Expr":
        return Expr("binary", "bool", op, self, as_expr(other))

    def __lt__(self, other: Any) -> "Expr":
        return self._cmp("<", other)

    def __le__(self, other: Any) -> "Expr":
        return self._cmp("<=", other)

    def __gt__(self, other: Any) -> "Expr":
        return self._cmp(">", other)

    def __ge__(self, other: Any) -> "Expr":
        return self._cmp(">=", other)

    def __eq__(self, other: Any) -> "Expr":  # type: ignore[override]
        return self._cmp("==", other)

    def __ne__(self, other: Any) -> "Expr":  # type: ignore[override]
        return self._cmp("!=", other)

    # -- casts -----------------------------------------------------------------
    def cast_bool(self) -> "Expr":
        return Expr("cast", "bool", self)

    def cast_i64(self) -> "Expr":
        return Expr("cast", "i64", self)

    def cast_u64(self) -> "Expr":
        return Expr("cast", "u64", self)


def _emit(e: Expr, out: list[str]) -> None:
    """Token grammar (one token per field, operands in prefix order):

    Lb 0|1 | Li <i64> | Lu <u64> | P <ty> <index> | K <ty> <scalar ordinal> | G <tag id> | A <ty> <axis id> |
    Y <symbol id> | S <ty> <slot> | U <op> <e> | B <op> <e> <e> | T <e> <e> <e> | C <ty> <e>
    with <ty> one of b, i, u.
    """
    k = e.kind
    if k == "lit_bool":
        out += ["Lb", "1" if e.a else "0"]
    elif k == "lit_i64":
        v = int(e.a)
        if not -(1 << 63) <= v < (1 << 63):
            raise TypeError(f"integer literal out of the i64 range: {v}")
        out += ["Li", str(v)]
    elif k == "lit_u64":
        out += ["Lu", str(int(e.a) & _MASK)]
    elif k == "task_param":
        out += ["P", _TYPE_CODE[e.type], str(int(e.a))]
    elif k == "kernel_scalar":
        out += ["K", _TYPE_CODE[e.type], str(int(e.a))]
    elif k == "task_tag_u64":
        out += ["G", str(int(e.a) & _MASK)]
    elif k == "axis_var":
        out += ["A", _TYPE_CODE[e.type], str(int(e.a) & _MASK)]
    elif k == "symbol_u64":
        out += ["Y", str(int(e.a) & _MASK)]
    elif k in ("slot_u64", "slot_i64", "slot_bool"):
        out += ["S", _TYPE_CODE[e.type], str(int(e.a))]
    elif k == "unary":
        out += ["U", str(e.a)]
        _emit(as_expr(e.b), out)
    elif k == "binary":
        out += ["B", str(e.a)]
        _emit(as_expr(e.b), out)
        _emit(as_expr(e.c), out)
    elif k == "ternary":
        out.append("T")
        for x in (e.a, e.b, e.c):
            _emit(as_expr(x), out)
    elif k == "cast":
        out += ["C", _TYPE_CODE[e.type]]
        _emit(as_expr(e.a), out)
    else:
        raise TypeError(f"Unsupported Expr kind: {k}")


def as_expr(x: Any) -> Expr:
    """``x`` as an Expr: Expr unchanged, bool -> lit_bool, int -> lit_i64."""
    if isinstance(x, Expr):
        return x
    if isinstance(x, bool):
        return Expr("lit_bool", "bool", x)
    if isinstance(x, int):
        return Expr("lit_i64", "i64", x)
    raise TypeError(f"Cannot convert to ScalarExpr: {x!r}")


class _Params:
    def __getitem__(self, i: int) -> Expr:
        return Expr("task_param", "i64", int(i))


class _Tags:
    def __getitem__(self, name: str) -> Expr:
        return Expr("task_tag_u64", "u64", fnv1a_64(str(name)))


class TaskExpr:
    """Stand-in task handed to schedule lambdas: ``t.params[i]``, ``t.tags[name]``, ``t.get(axis)``."""

    def __init__(self):
        self.params = _Params()
        self.tags = _Tags()

    def get(self, axis_name: str, default: int = 0) -> Expr:
        del default
        return axis(axis_name)


def trace_task_fn(fn: Callable[[TaskExpr], Any]) -> Expr:
    """Run ``fn`` on a TaskExpr to obtain its symbolic expression."""
    return as_expr(fn(TaskExpr()))


def symbol_u64(name: str) -> Expr:
    return Expr("symbol_u64", "u64", fnv1a_64(str(name)))


def slot_u64(i: int) -> Expr:
    return Expr("slot_u64", "u64", int(i))


def slot_i64(i: int) -> Expr:
    return Expr("slot_i64", "i64", int(i))


def slot_bool(i: int) -> Expr:
    return Expr("slot_bool", "bool", int(i))


def axis(name: str) -> Expr:
    """The enclosing loop variable called ``name`` (P(), P.seq or P.sel), as i64."""
    return Expr("axis_var", "i64", fnv1a_64(str(name)))


def task_param(index: int) -> Expr:
    return Expr("task_param", "i64", int(index))
