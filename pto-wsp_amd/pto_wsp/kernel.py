"""Tile-language tracer: ``pto.*`` records typed SSA ops into a ``KernelIR``.

Mirrors the reference tracer (``python/pto_wsp/kernel.py``):

* ``Tile[r, c]`` defaults to F16, ``Tile[r, c, dt]`` sets the dtype (kernel.py:98-110).
* ``ValueId`` numbers values 1, 2, ... per trace, parameters first (kernel.py:123-134).
* Elementwise results take operand 0's dtype and shape (kernel.py:306-310).
* Row reductions give ``(rows, 1)``; F16 inputs reduce to F32 (kernel.py:488-513).
* Matmul gives ``(a.rows, b.cols)``; F16@F16 accumulates to F32 (kernel.py:565-591).

One deliberate extension: BF16@BF16 also accumulates to F32.  The reference
types it as BF16 (its C++ emitter rejects BF16 altogether,
``src/python/pto_codegen.cpp:77-90``); MFMA accumulates bf16 products in fp32,
and the configurations this backend targets store fp32 results.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Any, Optional, Union

from pto_wsp.types import DType, Location


@dataclass(frozen=True)
class TileType:
    rows: Union[int, str]
    cols: Union[int, str]
    dtype: DType
    location: Location = Location.UB


@dataclass(frozen=True)
class ScalarType:
    dtype: DType


class Tile:
    """``Tile[rows, cols]`` (F16) or ``Tile[rows, cols, dtype]``."""

    def __class_getitem__(cls, args):
        if not isinstance(args, tuple):
            args = (args,)
        if len(args) == 2:
            return TileType(args[0], args[1], DType.F16)
        if len(args) == 3:
            return TileType(args[0], args[1], args[2])
        raise TypeError(f"Tile expects 2-3 args, got {len(args)}")


class Scalar:
    """``Scalar[dtype]``: a scalar kernel parameter."""

    def __class_getitem__(cls, dtype):
        return ScalarType(dtype)


class ValueId:
    _counter = 0

    @classmethod
    def next(cls) -> int:
        cls._counter += 1
        return cls._counter

    @classmethod
    def reset(cls) -> None:
        cls._counter = 0


@dataclass
class Value:
    id: int
    dtype: DType
    shape: Optional[tuple] = None
    location: Location = Location.UB
    debug_name: Optional[str] = None

    @classmethod
    def tile(cls, rows: int, cols: int, dtype: DType = DType.F16,
             location: Location = Location.UB, name: str | None = None) -> "Value":
        return cls(ValueId.next(), dtype, (rows, cols), location, name)

    @classmethod
    def scalar(cls, dtype: DType = DType.F32, name: str | None = None) -> "Value":
        return cls(ValueId.next(), dtype, None, Location.UB, name)

    def __repr__(self) -> str:
        return f"Value({self.debug_name}:{self.id})" if self.debug_name else f"Value({self.id})"


class OpKind(Enum):
    Load = auto()
    Store = auto()
    Alloc = auto()
    Add = auto()
    Sub = auto()
    Mul = auto()
    Div = auto()
    Max = auto()
    Min = auto()
    Neg = auto()
    Abs = auto()
    Exp = auto()
    Log = auto()
    Sqrt = auto()
    Rsqrt = auto()
    Tanh = auto()
    Sigmoid = auto()
    Relu = auto()
    Gelu = auto()
    Silu = auto()
    RowSum = auto()
    RowMax = auto()
    RowMean = auto()
    ColSum = auto()
    ColMax = auto()
    RowBroadcastAdd = auto()
    RowBroadcastMul = auto()
    RowExpandMul = auto()
    ColBroadcastAdd = auto()
    ColBroadcastMul = auto()
    Matmul = auto()
    Constant = auto()
    Sin = auto()
    Cos = auto()
    ForBegin = auto()
    ForEnd = auto()
    IfBegin = auto()
    IfEnd = auto()
    IotaU32 = auto()
    TSort32 = auto()
    ExtractTopkIndices = auto()
    # Extensions carrying the PTO-ISA kernels of pto_wsp.ptoisa_jit: TMOV, the
    # top-k index store and an explicit cycle-model increment.
    TMov = auto()
    StoreTopkIndices = auto()
    CpuSimAddCycles = auto()


@dataclass
class Op:
    kind: OpKind
    result: Optional[Value]
    operands: list
    attrs: dict = field(default_factory=dict)

    def __repr__(self) -> str:
        args = ", ".join(f"v{v.id}" for v in self.operands)
        if self.result is not None:
            return f"v{self.result.id} = {self.kind.name}({args})"
        return f"{self.kind.name}({args})"


@dataclass
class KernelIR:
    name: str
    params: list
    ops: list = field(default_factory=list)
    schedule_hints: dict = field(default_factory=dict)

    def add_op(self, kind: OpKind, operands: list, result: Optional[Value] = None, **attrs):
        self.ops.append(Op(kind, result, list(operands), dict(attrs)))
        return result

    def dump(self) -> str:
        lines = [f"@kernel {self.name}("]
        lines += [f"  {n}: v{v.id}" for n, v in self.params]
        lines.append(") {")
        lines += [f"  {op}" for op in self.ops]
        lines.append("}")
        return "\n".join(lines)


def _reduced_dtype(dt: DType) -> DType:
    return DType.F32 if dt == DType.F16 else dt


class _TileLanguage:
    """The ``pto`` namespace.  Every call appends one op to the kernel being traced."""

    def __init__(self) -> None:
        self._current_ir: Optional[KernelIR] = None

    # -- helpers -----------------------------------------------------------
    def _ir(self) -> KernelIR:
        if self._current_ir is None:
            raise RuntimeError("pto.* must be used inside a @kernel function")
        return self._current_ir

    def _elementwise(self, kind: OpKind, *operands: Value) -> Value:
        ir = self._ir()
        first = operands[0]
        out = Value(ValueId.next(), first.dtype, first.shape)
        ir.add_op(kind, list(operands), out)
        return out

    def _row_reduce(self, kind: OpKind, x: Value) -> Value:
        ir = self._ir()
        rows = x.shape[0] if x.shape else 1
        out = Value(ValueId.next(), _reduced_dtype(x.dtype), (rows, 1))
        ir.add_op(kind, [x], out)
        return out

    def _col_reduce(self, kind: OpKind, x: Value) -> Value:
        ir = self._ir()
        cols = x.shape[1] if x.shape else 1
        out = Value(ValueId.next(), _reduced_dtype(x.dtype), (1, cols))
        ir.add_op(kind, [x], out)
        return out

    # -- memory ------------------------------------------------------------
    def alloc(self, shape: tuple, dtype: DType = DType.F16, location: Location = Location.UB) -> Value:
        ir = self._ir()
        out = Value.tile(shape[0], shape[1], dtype, location)
        ir.add_op(OpKind.Alloc, [], out, shape=tuple(shape))
        return out

    def load(self, src: Value, offset: tuple = (0, 0), mask: Optional[Value] = None) -> Value:
        ir = self._ir()
        rows = src.shape[0] if src.shape else 32
        cols = src.shape[1] if src.shape else 128
        out = Value.tile(rows, cols, src.dtype)
        ir.add_op(OpKind.Load, [src] if mask is None else [src, mask], out, offset=tuple(offset))
        return out

    def store(self, dst: Value, src: Value, offset: tuple = (0, 0), mask: Optional[Value] = None) -> None:
        ir = self._ir()
        ir.add_op(OpKind.Store, [dst, src] if mask is None else [dst, src, mask], None, offset=tuple(offset))

    # -- binary ------------------------------------------------------------
    def add(self, a: Value, b: Value) -> Value:
        return self._elementwise(OpKind.Add, a, b)

    def sub(self, a: Value, b: Value) -> Value:
        return self._elementwise(OpKind.Sub, a, b)

    def mul(self, a: Value, b: Value) -> Value:
        return self._elementwise(OpKind.Mul, a, b)

    def div(self, a: Value, b: Value) -> Value:
        return self._elementwise(OpKind.Div, a, b)

    def maximum(self, a: Value, b: Value) -> Value:
        return self._elementwise(OpKind.Max, a, b)

    def minimum(self, a: Value, b: Value) -> Value:
        return self._elementwise(OpKind.Min, a, b)

    def max(self, a: Value, b: Value) -> Value:
        return self.maximum(a, b)

    def min(self, a: Value, b: Value) -> Value:
        return self.minimum(a, b)

    # -- unary -------------------------------------------------------------
    def exp(self, x: Value) -> Value:
        return self._elementwise(OpKind.Exp, x)

    def log(self, x: Value) -> Value:
        return self._elementwise(OpKind.Log, x)

    def sqrt(self, x: Value) -> Value:
        return self._elementwise(OpKind.Sqrt, x)

    def rsqrt(self, x: Value) -> Value:
        return self._elementwise(OpKind.Rsqrt, x)

    def tanh(self, x: Value) -> Value:
        return self._elementwise(OpKind.Tanh, x)

    def sigmoid(self, x: Value) -> Value:
        return self._elementwise(OpKind.Sigmoid, x)

    def relu(self, x: Value) -> Value:
        return self._elementwise(OpKind.Relu, x)

    def gelu(self, x: Value) -> Value:
        return self._elementwise(OpKind.Gelu, x)

    def silu(self, x: Value) -> Value:
        return self._elementwise(OpKind.Silu, x)

    def neg(self, x: Value) -> Value:
        return self._elementwise(OpKind.Neg, x)

    def abs(self, x: Value) -> Value:
        return self._elementwise(OpKind.Abs, x)

    def sin(self, x: Value) -> Value:
        return self._elementwise(OpKind.Sin, x)

    def cos(self, x: Value) -> Value:
        return self._elementwise(OpKind.Cos, x)

    # -- slice / interleave / broadcast (RoPE helpers) ----------------------
    # The reference traces these as Constant ops that carry their operands
    # and a marker attr (python/pto_wsp/kernel.py:631-685); its lowering gives
    # a tile-shaped Constant no compute, so compiling a kernel that uses them
    # raises CompileError here.  The result shapes follow the reference,
    # including its (32, 64) / (32, 128) default for a scalar operand.
    def slice_even(self, x: Value) -> Value:
        """x[:, 0::2]: even-indexed elements along the last dimension."""
        return self._half_slice(x, "even")

    def slice_odd(self, x: Value) -> Value:
        """x[:, 1::2]: odd-indexed elements along the last dimension."""
        return self._half_slice(x, "odd")

    def _half_slice(self, x: Value, which: str) -> Value:
        ir = self._ir()
        shape = (x.shape[0], x.shape[1] // 2) if x.shape else (32, 64)
        out = Value(ValueId.next(), x.dtype, shape)
        ir.add_op(OpKind.Constant, [x], out, slice_type=which)
        return out

    def interleave(self, a: Value, b: Value) -> Value:
        """Even elements from a, odd elements from b, along the last dimension."""
        ir = self._ir()
        shape = (a.shape[0], a.shape[1] * 2) if a.shape else (32, 128)
        out = Value(ValueId.next(), a.dtype, shape)
        ir.add_op(OpKind.Constant, [a, b], out, op_type="interleave")
        return out

    def broadcast(self, x: Value, shape: tuple) -> Value:
        """x broadcast to `shape`."""
        ir = self._ir()
        out = Value(ValueId.next(), x.dtype, tuple(shape))
        ir.add_op(OpKind.Constant, [x], out, broadcast_shape=tuple(shape))
        return out

    # -- reductions --------------------------------------------------------
    def rowsum(self, x: Value) -> Value:
        return self._row_reduce(OpKind.RowSum, x)

    def rowmax(self, x: Value) -> Value:
        return self._row_reduce(OpKind.RowMax, x)

    def rowmean(self, x: Value) -> Value:
        return self._row_reduce(OpKind.RowMean, x)

    def colsum(self, x: Value) -> Value:
        return self._col_reduce(OpKind.ColSum, x)

    def colmax(self, x: Value) -> Value:
        return self._col_reduce(OpKind.ColMax, x)

    # -- broadcasts (recorded; lowered only through Mul/Add/... shapes) ----
    def rowmul(self, tile: Value, vec: Value) -> Value:
        ir = self._ir()
        out = Value(ValueId.next(), tile.dtype, tile.shape)
        ir.add_op(OpKind.RowBroadcastMul, [tile, vec], out)
        return out

    def rowadd(self, tile: Value, vec: Value) -> Value:
        ir = self._ir()
        out = Value(ValueId.next(), tile.dtype, tile.shape)
        ir.add_op(OpKind.RowBroadcastAdd, [tile, vec], out)
        return out

    def colmul(self, tile: Value, vec: Value) -> Value:
        ir = self._ir()
        out = Value(ValueId.next(), tile.dtype, tile.shape)
        ir.add_op(OpKind.ColBroadcastMul, [tile, vec], out)
        return out

    def coladd(self, tile: Value, vec: Value) -> Value:
        ir = self._ir()
        out = Value(ValueId.next(), tile.dtype, tile.shape)
        ir.add_op(OpKind.ColBroadcastAdd, [tile, vec], out)
        return out

    # -- matrix ------------------------------------------------------------
    def matmul(self, a: Value, b: Value, acc: Optional[Value] = None) -> Value:
        ir = self._ir()
        rows = a.shape[0] if a.shape else 32
        cols = b.shape[1] if b.shape else 32
        if a.dtype == b.dtype and a.dtype in (DType.F16, DType.BF16):
            out_dtype = DType.F32
        else:
            out_dtype = a.dtype
        if acc is not None and acc.dtype != out_dtype:
            raise TypeError(f"matmul acc dtype mismatch: acc={acc.dtype} out={out_dtype}")
        out = Value(ValueId.next(), out_dtype, (rows, cols))
        ir.add_op(OpKind.Matmul, [a, b] if acc is None else [a, b, acc], out)
        return out

    # -- PTO-ISA helpers (reference kernel.py:689-724) ---------------------
    def iota_u32(self, cols: int) -> Value:
        """A [1, cols] u32 tile holding 0 .. cols-1."""
        ir = self._ir()
        c = int(cols)
        if c <= 0:
            raise ValueError("iota_u32: cols must be > 0")
        out = Value(ValueId.next(), DType.U32, (1, c))
        ir.add_op(OpKind.IotaU32, [], out, cols=c)
        return out

    def tsort32(self, scores: Value, idx: Value) -> Value:
        """TSORT32: the 32 (score, index) pairs sorted by descending score, as an f32 [1, 64]
        tile of interleaved pairs (index stored as an f32 value)."""
        ir = self._ir()
        if scores.shape != (1, 32) or scores.dtype != DType.F32:
            raise ValueError("tsort32: scores must be Tile[1,32,F32]")
        if idx.shape != (1, 32) or idx.dtype != DType.U32:
            raise ValueError("tsort32: idx must be Tile[1,32,U32]")
        out = Value(ValueId.next(), DType.F32, (1, 64))
        ir.add_op(OpKind.TSort32, [scores, idx], out)
        return out

    def extract_topk_indices(self, pairs: Value, k: int) -> Value:
        """The indices of the first k pairs of a tsort32 result, as an i32 [1, k] tile."""
        ir = self._ir()
        kk = int(k)
        if pairs.shape != (1, 64) or pairs.dtype != DType.F32:
            raise ValueError("extract_topk_indices: pairs must be Tile[1,64,F32] from tsort32")
        if kk <= 0 or kk > 32:
            raise ValueError("extract_topk_indices: k must be in [1,32]")
        out = Value(ValueId.next(), DType.I32, (1, kk))
        ir.add_op(OpKind.ExtractTopkIndices, [pairs], out, k=kk)
        return out

    # -- scalars -----------------------------------------------------------
    def constant(self, value: float, dtype: DType = DType.F32) -> Value:
        ir = self._ir()
        out = Value.scalar(dtype, name=f"const_{value}")
        ir.add_op(OpKind.Constant, [], out, value=value)
        return out


pto = _TileLanguage()
tl = pto
