"""Axis types, dtypes and tensor views of the PTO-WSP authoring API.

Behaviour mirrors the reference frontend (``python/pto_wsp/types.py``):

* ``Dense[n]()``   static-extent axis                 (types.py:14-33)
* ``DenseDyn(n)``  extent bound at run time by name    (types.py:36-47)
* ``Ragged``       flattened sum-of-lengths axis       (types.py:50-68)
* ``Sparse``       CSR axis for ``P.sel``              (types.py:71-96)
* ``Symbol``       run-time scalar symbol              (types.py:99-116)
* ``DType``        element types                        (types.py:119-132)
* ``Tensor``       base tensor or a view recording symbolic index expressions
                   (types.py:365-460): indexing drops leading dimensions and
                   appends to ``index_exprs``; the base is kept for codegen.

A ``Tensor`` holds its storage in ``data``: a numpy array (host memory; the
HIP backend stages it through HBM) or a ``torch`` tensor already resident on
the GPU (used in place, no copy).  Element strides are taken from the
storage object, so transposed or otherwise strided views work unchanged.
"""

from __future__ import annotations

from enum import Enum
from typing import Any, Generic, TypeVar

N = TypeVar("N", bound=int)


class Dense(Generic[N]):
    """Axis with an extent fixed when the workload is built: ``Dense[8]()``."""

    _size: int = 0

    def __class_getitem__(cls, n: int) -> type:
        extent = int(n)

        class _DenseN(Dense):
            _size = extent

        _DenseN.__name__ = f"Dense[{extent}]"
        return _DenseN

    def __init__(self) -> None:
        pass

    @property
    def size(self) -> int:
        return self._size

    def __repr__(self) -> str:
        return f"Dense[{self._size}]()"


class DenseDyn:
    """Axis whose extent is read at run time.

    ``DenseDyn(size)`` is the reference's axis (``python/pto_wsp/types.py:36-47``):
    one extent per loop variable name, rebound with ``Program.set_axis_sizes``;
    ``size`` is the default until then.

    Extension (per-outer extents, e.g. pages per sequence of a paged KV cache):
    ``DenseDyn(max_size, extent=N[b])`` takes the extent of each loop instance
    from one element of an I32 tensor, indexed by enclosing loop variables.
    ``max_size`` is then only an upper bound used for sizing.
    """

    def __init__(self, size: int, extent=None) -> None:
        self._size = int(size)
        if extent is not None:
            from_tensor = getattr(extent, "base", None)
            if from_tensor is None or getattr(from_tensor, "dtype", None) != DType.I32:
                raise TypeError("DenseDyn extent must be an element view of an I32 tensor")
            if tuple(extent.shape) != ():
                raise TypeError(f"DenseDyn extent must select one element (view shape {tuple(extent.shape)})")
        self.extent_view = extent

    @property
    def size(self) -> int:
        return self._size

    def __repr__(self) -> str:
        if self.extent_view is not None:
            return f"DenseDyn({self._size}, extent={self.extent_view!r})"
        return f"DenseDyn({self._size})"


class Ragged:
    """Variable-length axis: iterates the flattened index ``0 .. sum(lengths)-1``.

    The extent is bound at run time through the symbols ``outer_<id>`` (u64)
    and ``lengths_<id>`` (int32 array), exactly like the reference lowering
    (``src/python/pto_codegen.cpp:2321-2340``).
    """

    def __init__(self, outer_size: int, lengths: list[int]) -> None:
        self._outer_size = int(outer_size)
        self._lengths = [int(x) for x in lengths]

    @property
    def outer_size(self) -> int:
        return self._outer_size

    def length(self, idx: int) -> int:
        return self._lengths[idx]

    def total(self) -> int:
        return sum(self._lengths[: self._outer_size])

    @property
    def size(self) -> int:
        return self.total()


class Sparse:
    """CSR iteration space (``indptr``/``indices``) for ``P.sel``."""

    def __init__(self, outer_size: int, indptr: list[int], indices: list[int]) -> None:
        self._outer_size = int(outer_size)
        self._indptr = [int(x) for x in indptr]
        self._indices = [int(x) for x in indices]

    @property
    def outer_size(self) -> int:
        return self._outer_size

    @property
    def indices(self) -> list[int]:
        return list(self._indices)

    def nnz(self) -> int:
        return self._indptr[self._outer_size]

    def row_nnz(self, row: int) -> int:
        return self._indptr[row + 1] - self._indptr[row]

    def __getitem__(self, row: int) -> list[int]:
        return self._indices[self._indptr[row]: self._indptr[row + 1]]


class Symbol:
    """Scalar kernel argument looked up by name in the program's symbol table."""

    def __init__(self, sym: str) -> None:
        self.sym = str(sym)

    def __repr__(self) -> str:
        return f"Symbol({self.sym!r})"


class DType(Enum):
    F16 = "f16"
    BF16 = "bf16"
    F32 = "f32"
    F64 = "f64"
    I8 = "i8"
    I16 = "i16"
    I32 = "i32"
    I64 = "i64"
    U8 = "u8"
    U16 = "u16"
    U32 = "u32"
    U64 = "u64"


DTYPE_NBYTES = {
    DType.F16: 2, DType.BF16: 2, DType.F32: 4, DType.F64: 8,
    DType.I8: 1, DType.I16: 2, DType.I32: 4, DType.I64: 8,
    DType.U8: 1, DType.U16: 2, DType.U32: 4, DType.U64: 8,
}


class Location(Enum):
    Global = "global"
    L2 = "l2"
    UB = "ub"
    L1 = "l1"


class Tensor:
    """A base tensor, or a view of one reached through ``__getitem__``.

    ``X[b][t]`` is a view whose ``base`` is ``X`` and whose ``index_exprs``
    are ``(b, t)``; its shape is ``X.shape[2:]``.  Index expressions may be
    integers, loop variables, affine combinations of loop variables, or an
    element of an int32 index tensor (``PT[b][p]``, an indirect index).
    """

    def __init__(
        self,
        data: Any,
        shape: tuple[int, ...],
        dtype: DType,
        location: Location = Location.Global,
        layout: Any = None,
        base: "Tensor | None" = None,
        index_exprs: tuple[Any, ...] = (),
    ) -> None:
        self.data = data
        self.shape = tuple(int(d) for d in shape)
        self.dtype = dtype
        self.location = location
        self.layout = layout
        self._base: Tensor = base if base is not None else self
        self._index_exprs: tuple[Any, ...] = tuple(index_exprs)

    @property
    def base(self) -> "Tensor":
        return self._base

    @property
    def index_exprs(self) -> tuple[Any, ...]:
        return self._index_exprs

    def __getitem__(self, idx: Any) -> "Tensor":
        from pto_wsp.builder import get_current_builder

        indices = idx if isinstance(idx, tuple) else (idx,)
        builder = get_current_builder()
        if builder is not None:
            builder.check_tensor_access(self, indices)
        if not self.shape:
            return self
        drop = min(len(indices), len(self.shape))
        return Tensor(
            data=self.data,
            shape=self.shape[drop:],
            dtype=self.dtype,
            location=self.location,
            layout=self.layout,
            base=self._base,
            index_exprs=self._index_exprs + tuple(indices),
        )

    def nbytes(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n * DTYPE_NBYTES.get(self.dtype, 4) if self.shape else 0

    def __repr__(self) -> str:
        if self._base is self:
            return f"Tensor(shape={self.shape}, dtype={self.dtype.value})"
        return f"TensorView(base={self._base.shape}, index={self._index_exprs}, shape={self.shape})"
