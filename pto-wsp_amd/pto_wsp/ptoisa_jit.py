"""``@ptoisa_kernel``: kernels written with PTO-ISA instruction names.

The reference (``python/pto_wsp/ptoisa_jit.py:124-559``) traces ``ptoisa.*``
calls at decoration time into a C++ kernel body (``cpp_src``) of PTO-ISA
wrapper calls.  That tile library is not part of this target, so each
instruction is traced into the kernel IR instead and runs on the device like
any ``pto.*`` kernel (the tile program):

* ``tload`` / ``tstore``      -> Load / Store of a parameter tile;
* ``TADD`` .. ``TMIN``        -> the elementwise ops (equal shapes and dtypes,
  checked as the reference checks them);
* ``TROWEXPAND*`` / ``TCOLEXPAND*`` -> the same ops with a [R,1] / [1,C]
  right operand (row / column broadcast);
* ``TADDS`` .. ``TMINS``      -> the op with a scalar: a number (a constant of
  the tile's dtype) or a ``Scalar[...]`` parameter;
* ``TEXP`` / ``TRSQRT``       -> Exp / Rsqrt;
* ``TMOV``                    -> TMov (a tile copy);
* ``TSORT32``, ``iota_u32``   -> TSort32, IotaU32 (as ``pto.tsort32`` / ``pto.iota_u32``);
* ``store_topk_indices_i32``  -> StoreTopkIndices (the first k pair indices
  written along row 0 of the output tile);
* ``cpu_sim_add_cycles(n)``   -> CpuSimAddCycles: an integer, or a ``Scalar`` parameter or
  a C expression string over the kernel's scalar parameters, which the cycle
  model evaluates per task with that task's scalar arguments.

The cycle model charges what the reference's wrappers charge
(``include/pto/wsp/codegen/abi/ptoisa_bridge.hpp:54-303``): valid rows x cols
per TLOAD / TSTORE / TMOV / elementwise op, 5 per element of a TSORT32 source,
nothing for the helper loops (iota, top-k store), plus ``cpu_sim_add_cycles``.
``cpp_includes`` name host headers and are refused.
"""

from __future__ import annotations

from typing import Any, Callable, Optional

import re

from pto_wsp.builder import Kernel, extract_kernel_params
from pto_wsp.scalar_expr import Expr
from pto_wsp.kernel import KernelIR, OpKind, ScalarType, TileType, Value, ValueId, pto
from pto_wsp.types import DType

_BINARY = {"TADD": "add", "TSUB": "sub", "TMUL": "mul", "TDIV": "div", "TMAX": "max", "TMIN": "min"}
_ROWEXPAND = {"TROWEXPANDADD": "add", "TROWEXPANDSUB": "sub", "TROWEXPANDMUL": "mul", "TROWEXPANDDIV": "div",
              "TROWEXPANDMAX": "max", "TROWEXPANDMIN": "min"}
_COLEXPAND = {"TCOLEXPANDSUB": "sub", "TCOLEXPANDMUL": "mul", "TCOLEXPANDDIV": "div"}
_SCALAR = {"TADDS": "add", "TSUBS": "sub", "TMULS": "mul", "TDIVS": "div", "TMAXS": "max", "TMINS": "min"}
_UNARY = {"TEXP": "exp", "TRSQRT": "rsqrt"}


class _PtoisaNamespace:
    """Authoring surface for PTO-ISA kernels; usable only while a ``@ptoisa_kernel`` traces."""

    def _ir(self) -> KernelIR:
        ir = pto._current_ir
        if ir is None:
            raise RuntimeError("ptoisa ops can only be used inside @ptoisa_kernel during tracing")
        return ir

    def _param_tile(self, v: Any, what: str) -> Value:
        ir = self._ir()
        if not isinstance(v, Value) or v.shape is None or not any(p is v for _, p in ir.params):
            raise TypeError(f"{what} expects a kernel param tile (In/Out[Tile[...]])")
        return v

    def _tile(self, v: Any, what: str) -> Value:
        """A tile produced inside the kernel (tload or an instruction): param tiles
        are read through ``tload`` first, as in the reference tracer."""
        ir = self._ir()
        if not isinstance(v, Value) or v.shape is None or any(p is v for _, p in ir.params):
            raise TypeError(f"{what}: expects a tile value")
        return v

    # -- memory -----------------------------------------------------------
    def tload(self, src: Value) -> Value:
        return pto.load(self._param_tile(src, "ptoisa.tload"))

    def tstore(self, dst: Value, src: Value) -> None:
        d, v = self._param_tile(dst, "ptoisa.tstore"), self._tile(src, "ptoisa.tstore")
        if d.shape != v.shape or d.dtype != v.dtype:
            raise ValueError(f"ptoisa.tstore: a {v.shape} {v.dtype.value} tile into a {d.shape} {d.dtype.value} param")
        pto.store(d, v)

    # -- helpers ----------------------------------------------------------
    def iota_u32(self, cols: int) -> Value:
        self._ir()
        return pto.iota_u32(cols)

    def store_topk_indices_i32(self, dst: Value, pairs: Value, k: int) -> None:
        ir = self._ir()
        d = self._param_tile(dst, "store_topk_indices_i32")
        p = self._tile(pairs, "store_topk_indices_i32")
        kk = int(k)
        if p.shape != (1, 64) or p.dtype != DType.F32:
            raise ValueError("store_topk_indices_i32: pairs must be the Tile[1,64,F32] result of TSORT32")
        if not 1 <= kk <= min(32, d.shape[1]):
            raise ValueError(f"store_topk_indices_i32: k={kk} must be in [1, {min(32, d.shape[1])}]")
        if d.dtype not in (DType.I32, DType.I64):
            raise ValueError("store_topk_indices_i32: the output tile must be I32 or I64")
        ir.add_op(OpKind.StoreTopkIndices, [d, p], None, k=kk)

    def cpu_sim_add_cycles(self, cycles: Any) -> None:
        """add_cycles((uint64_t)(cycles)) per task: an integer, a ``Scalar[...]`` parameter, or
        a C expression string over the kernel's scalar parameters (reference
        ptoisa_jit.py:206-208, 458-463), evaluated per task by the cycle model."""
        ir = self._ir()
        scalars = [(n, v) for n, v in ir.params if v.shape is None]
        if isinstance(cycles, Value) and cycles.shape is None:
            ords = [i for i, (_, v) in enumerate(scalars) if v is cycles]
            if not ords:
                raise TypeError("cpu_sim_add_cycles: the value must be a Scalar[...] parameter of the kernel")
            expr = _scalar_ref(ords[0], cycles.dtype)
            ir.add_op(OpKind.CpuSimAddCycles, [], None, cycles_expr=expr.to_text())
            return
        if isinstance(cycles, str):
            env = {n: _scalar_ref(i, v.dtype) for i, (n, v) in enumerate(scalars)}
            expr = parse_c_expr(cycles, env)
            ir.add_op(OpKind.CpuSimAddCycles, [], None, cycles_expr=expr.to_text())
            return
        if isinstance(cycles, bool) or not isinstance(cycles, int):
            raise TypeError("cpu_sim_add_cycles: expects an int, a Scalar parameter or a C expression string")
        if cycles < 0:
            raise ValueError("cpu_sim_add_cycles: the cycle count must be >= 0")
        ir.add_op(OpKind.CpuSimAddCycles, [], None, cycles=int(cycles))

    # -- instructions -----------------------------------------------------
    def _bin(self, name: str, a: Any, b: Any) -> Value:
        a, b = self._tile(a, name), self._tile(b, name)
        if a.shape != b.shape or a.dtype != b.dtype:
            raise ValueError(f"{name}: shape/dtype mismatch: {a.shape} {a.dtype.value} vs {b.shape} {b.dtype.value}")
        return getattr(pto, _BINARY[name])(a, b)

    def _expand(self, name: str, a: Any, b: Any) -> Value:
        a, b = self._tile(a, name), self._tile(b, name)
        rows, cols = a.shape
        want = (rows, 1) if name in _ROWEXPAND else (1, cols)
        if b.shape != want or b.dtype != a.dtype:
            raise ValueError(f"{name}: the broadcast operand must be a {want} tile of {a.dtype.value} (got {b.shape})")
        return getattr(pto, (_ROWEXPAND if name in _ROWEXPAND else _COLEXPAND)[name])(a, b)

    def _scalar_op(self, name: str, a: Any, s: Any) -> Value:
        a = self._tile(a, name)
        if isinstance(s, Value) and s.shape is None:
            sv = s
        elif isinstance(s, (int, float)) and not isinstance(s, bool):
            # (elem)(scalar): an integer tile truncates the number.
            sv = pto.constant(float(s) if a.dtype.value.startswith(("f", "bf")) else int(s), a.dtype)
        else:
            raise TypeError(f"{name}: the scalar must be a number or a Scalar[...] parameter (got {s!r})")
        return getattr(pto, _SCALAR[name])(a, sv)

    def TMOV(self, a: Any) -> Value:  # noqa: N802
        a = self._tile(a, "TMOV")
        out = Value(ValueId.next(), a.dtype, a.shape)
        self._ir().add_op(OpKind.TMov, [a], out)
        return out

    def TSORT32(self, src: Any, idx: Any) -> Value:  # noqa: N802
        src, idx = self._tile(src, "TSORT32"), self._tile(idx, "TSORT32")
        if src.shape != (1, 32):
            raise ValueError("TSORT32 v9: requires src tile shape [1,32]")
        if idx.shape != (1, 32) or idx.dtype != DType.U32:
            raise ValueError("TSORT32 v9: requires idx tile shape [1,32] dtype u32")
        if src.dtype != DType.F32:
            raise ValueError("TSORT32 v9: requires src dtype f32")
        return pto.tsort32(src, idx)

    def __getattr__(self, name: str) -> Any:
        if name in _BINARY:
            return lambda a, b: self._bin(name, a, b)
        if name in _ROWEXPAND or name in _COLEXPAND:
            return lambda a, b: self._expand(name, a, b)
        if name in _SCALAR:
            return lambda a, s: self._scalar_op(name, a, s)
        if name in _UNARY:
            return lambda a: getattr(pto, _UNARY[name])(self._tile(a, name))
        raise AttributeError(name)


ptoisa = _PtoisaNamespace()


# -- C expressions of cycle counts --------------------------------------------
def _scalar_ref(ordinal: int, dtype: DType) -> Expr:
    """The task's value of scalar parameter `ordinal`, typed as its C counterpart promotes."""
    if dtype in (DType.I8, DType.I16, DType.I32, DType.I64):
        return Expr("kernel_scalar", "i64", int(ordinal))
    if dtype in (DType.U8, DType.U16, DType.U32, DType.U64):
        return Expr("kernel_scalar", "u64", int(ordinal))
    raise TypeError(f"cpu_sim_add_cycles: scalar parameters of dtype {dtype.value} cannot appear in a cycle count")


_C_TYPES = {
    "uint64_t": "u64", "size_t": "u64", "unsigned long long": "u64", "unsigned long": "u64",
    "int64_t": "i64", "long long": "i64", "long": "i64", "int": "i64", "int32_t": "i64", "bool": "bool",
}
_C_TOKEN = re.compile(r"\s*(?:(0[xX][0-9a-fA-F]+|\d+)([uUlL]*)|([A-Za-z_]\w*)|(<<|>>|<=|>=|==|!=|&&|\|\||[-+*/%<>&|^!~?:()]))")
_BINARY_PREC = [("||",), ("&&",), ("|",), ("^",), ("&",), ("==", "!="), ("<", "<=", ">", ">="), ("<<", ">>"),
                ("+", "-"), ("*", "/", "%")]


def _promote(t: str) -> str:
    return "i64" if t == "bool" else t


def parse_c_expr(src: str, env: dict) -> Expr:
    """Parses a C expression over integer literals (``u``/``l`` suffixes), the names in
    ``env`` (kernel scalar parameters), casts to the integer types of ``_C_TYPES``, unary
    ``- ! ~``, the binary operators of C and ``?:``.  int-typed values are evaluated as
    int64 (the same results wherever the C expression does not overflow int)."""
    toks = []
    pos = 0
    while pos < len(src):
        if src[pos:].strip() == "":
            break
        m = _C_TOKEN.match(src, pos)
        if not m:
            raise ValueError(f"cpu_sim_add_cycles: cannot parse {src[pos:]!r} in {src!r}")
        pos = m.end()
        if m.group(1) is not None:
            suffix = m.group(2).lower()
            if suffix not in ("", "u", "l", "ul", "lu", "ll", "ull", "llu"):
                raise ValueError(f"cpu_sim_add_cycles: bad literal suffix in {src!r}")
            toks.append(("num", int(m.group(1), 0), "u" in suffix))
        elif m.group(3) is not None:
            toks.append(("id", m.group(3)))
        else:
            toks.append(("op", m.group(4)))
    i = 0

    def peek(k=0):
        return toks[i + k] if i + k < len(toks) else ("end",)

    def take(op=None):
        nonlocal i
        t = peek()
        if op is not None and t != ("op", op):
            raise ValueError(f"cpu_sim_add_cycles: expected {op!r} in {src!r}")
        i += 1
        return t

    def cast_type():
        # "(" type-name ")" at the current position, or None.
        names, k = [], 1
        if peek() != ("op", "("):
            return None
        while peek(k)[0] == "id" and peek(k)[1] in ("unsigned", "long", "int", "uint64_t", "int64_t", "size_t",
                                                     "int32_t", "bool"):
            names.append(peek(k)[1])
            k += 1
        if not names or peek(k) != ("op", ")"):
            return None
        name = " ".join(names)
        if name not in _C_TYPES:
            raise ValueError(f"cpu_sim_add_cycles: unsupported cast to {name!r} in {src!r}")
        return _C_TYPES[name], k + 1

    def unary() -> Expr:
        nonlocal i
        c = cast_type()
        if c is not None:
            i += c[1]
            return Expr("cast", c[0], unary())
        t = peek()
        if t[0] == "op" and t[1] in ("-", "!", "~", "+"):
            take()
            x = unary()
            if t[1] == "+":
                return x
            return Expr("unary", "bool" if t[1] == "!" else _promote(x.type), t[1], x)
        if t == ("op", "("):
            take()
            x = ternary()
            take(")")
            return x
        if t[0] == "num":
            take()
            if t[2] or t[1] >= (1 << 63):
                return Expr("lit_u64", "u64", t[1] & ((1 << 64) - 1))
            return Expr("lit_i64", "i64", t[1])
        if t[0] == "id":
            take()
            if t[1] in ("true", "false"):
                return Expr("lit_bool", "bool", t[1] == "true")
            if t[1] not in env:
                raise ValueError(f"cpu_sim_add_cycles: {t[1]!r} is not a scalar parameter of the kernel ({src!r})")
            return env[t[1]]
        raise ValueError(f"cpu_sim_add_cycles: unexpected {t!r} in {src!r}")

    def binary(level: int) -> Expr:
        if level == len(_BINARY_PREC):
            return unary()
        lhs = binary(level + 1)
        while peek()[0] == "op" and peek()[1] in _BINARY_PREC[level]:
            op = take()[1]
            rhs = binary(level + 1)
            if op in ("==", "!=", "<", "<=", ">", ">=", "&&", "||"):
                t = "bool"
            elif op in ("<<", ">>"):
                t = _promote(lhs.type)
            else:
                t = "u64" if "u64" in (_promote(lhs.type), _promote(rhs.type)) else "i64"
            lhs = Expr("binary", t, op, lhs, rhs)
        return lhs

    def ternary() -> Expr:
        c = binary(0)
        if peek() == ("op", "?"):
            take()
            a = ternary()
            take(":")
            b = ternary()
            if a.type == b.type == "bool":
                t = "bool"
            else:
                t = "u64" if "u64" in (_promote(a.type), _promote(b.type)) else "i64"
            return Expr("ternary", t, c, a, b)
        return c

    e = ternary()
    if peek() != ("end",):
        raise ValueError(f"cpu_sim_add_cycles: trailing {peek()!r} in {src!r}")
    return e


def ptoisa_kernel(func: Callable | None = None, *, cpp_includes: Optional[list] = None) -> Any:
    """Define a kernel authored with PTO-ISA instruction calls (reference ptoisa_jit.py:510-559).

    The body is traced once at decoration time, so errors surface there as in
    the reference; the result is an ordinary ``Kernel`` used as
    ``name[axes](**views)`` inside workloads."""

    def decorator(fn: Callable) -> Kernel:
        if cpp_includes:
            raise ValueError("ptoisa_kernel: cpp_includes name host headers, which the hip_gfx950 target cannot include")
        for p in extract_kernel_params(fn):
            ok = (isinstance(p.inner_type, TileType) and p.shape is not None) or isinstance(p.inner_type, ScalarType)
            if not ok:
                raise TypeError(
                    f"ptoisa_kernel only supports Tile[...] and Scalar[...] params (got {p.name}: {p.inner_type!r})")
        k = Kernel(fn, ptoisa=True)
        k.trace()
        return k

    return decorator(func) if func is not None else decorator
