"""Python workload -> codegen module text.

Plays the role of ``workload_to_codegen_ir`` in the reference
(``python/pto_wsp/ir_bridge.py:112-139``), which builds a pybind ``ir::Module``
holding the tensor table, one ``CodegenKernelDef`` per kernel and the workload
tree with codegen bindings.  Here the same content is serialized to a small
line-oriented text module (format ``PTOWSP-MODULE 1``) that the C++ host
library parses; the C-ABI then needs only a ``const char*``.

Conversion rules kept from the reference:

* tensor table = unique base tensors in first-use order (:768-847);
* kernels sorted by name, each traced once (:127, :963-1017);
* DenseDyn loop axes are keyed by the loop variable name (:401-405);
* Ragged axes read the symbols ``outer_<id>`` / ``lengths_<id>`` (:179-183);
* axis args: loop var, string (FNV-1a-64 hash) or integer (:887-905);
* scalar args: Symbol (looked up by FNV-1a-64 id), loop var, f32 bits, i32, i64 (:908-944);
* a schedule is emitted only when ``Schedule.to_dict()`` is non-empty; the
  task window rides along with it (:129-131, :591-697).
"""

from __future__ import annotations

import inspect
import math
import struct
from dataclasses import dataclass
from typing import Any

from pto_wsp.errors import IRBridgeError
from pto_wsp.p_namespace import AffineIndex, LoopVar
from pto_wsp.scalar_expr import as_expr, trace_task_fn
from pto_wsp.types import DenseDyn, DType, Ragged, Sparse, Symbol, Tensor
from pto_wsp.workload import Workload, axis_extent

MODULE_MAGIC = "PTOWSP-MODULE 1"


def fnv1a_64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode("utf-8"):
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


_SAFE = set("ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789_.:-")


def enc(s: str) -> str:
    """Token-safe string: bytes outside ``[A-Za-z0-9_.:-]`` become ``%XX``; '' -> '%'."""
    if s == "":
        return "%"
    out = []
    for b in s.encode("utf-8"):
        c = chr(b)
        out.append(c if c in _SAFE else f"%{b:02X}")
    return "".join(out)


def dtype_str(dt: Any) -> str:
    v = getattr(dt, "value", str(dt))
    if v not in {d.value for d in DType} and v != "bool":
        raise IRBridgeError(f"Unsupported dtype for codegen: {dt!r}")
    return v


@dataclass(frozen=True)
class CodegenIRBuild:
    module: str
    tensors: list


class _Collector:
    def __init__(self) -> None:
        self.tensor_ids: dict[int, int] = {}
        self.tensors: list[Tensor] = []
        self.kernels: dict[str, Any] = {}
        self.bodies: dict[int, tuple] = {}  # id(loop node) -> (node, body workload)

    def body(self, node: Workload) -> Any:
        """The body workload of a loop node; a callable body (the functional
        primitives) is called once with the loop variable and the result kept."""
        kw = node._kwargs
        b = kw.get("body")
        if callable(b) and not isinstance(b, Workload):
            key = id(node)
            if key not in self.bodies:
                default = "e" if node._kind == "select" else "i"
                var = str(kw.get("var_name", default))
                self.bodies[key] = (node, b(LoopVar(var, kw.get("axis"))))
            return self.bodies[key][1]
        return b

    def collect(self, node: Any) -> None:
        if not isinstance(node, Workload):
            return
        kind, kw = node._kind, node._kwargs
        if kind == "task":
            k = kw.get("kernel")
            if k is not None and hasattr(k, "name"):
                self.kernels[str(k.name)] = k
            res = kw.get("resources", {})
            for v in (res.values() if isinstance(res, dict) else res):
                self._register(v)
        elif kind in ("parallel_for", "for_each"):
            self._register_axis(kw.get("axis"))
            self.collect(self.body(node))
        elif kind in ("combine", "sequential"):
            for c in kw.get("workloads", []) or []:
                self.collect(c)
        elif kind == "cond":
            self.collect(kw.get("then_workload"))
            self.collect(kw.get("else_workload"))
        elif kind == "select":
            self.collect(self.body(node))
        elif kind == "slot_load_u64":
            self._register(kw.get("tensor"))

    def _register(self, t: Any) -> None:
        if not isinstance(t, Tensor):
            return
        base = t.base
        if id(base) not in self.tensor_ids:
            self.tensor_ids[id(base)] = len(self.tensors)
            self.tensors.append(base)
        for e in t.index_exprs:
            if isinstance(e, Tensor):
                self._register(e)

    def _register_axis(self, axis: Any) -> None:
        bound = getattr(axis, "extent_view", None)
        if isinstance(bound, Tensor):
            self._register(bound)


class _Writer:
    def __init__(self, collector: _Collector) -> None:
        self.c = collector
        self.lines: list[str] = []

    def emit(self, *tokens: Any) -> None:
        self.lines.append(" ".join(str(t) for t in tokens))

    # -- index expressions ------------------------------------------------
    def index_expr(self, e: Any) -> str:
        if isinstance(e, LoopVar):
            return f"v {enc(e.name)}"
        if isinstance(e, AffineIndex):
            if not e.terms:
                return f"c {e.const}"
            terms = " ".join(f"{enc(n)} {c}" for n, c in sorted(e.terms.items()))
            return f"a {e.const} {len(e.terms)} {terms}"
        if isinstance(e, Tensor):
            base = e.base
            if base.dtype != DType.I32:
                raise IRBridgeError("indirect index tensors must be I32")
            if len(e.shape) != 0:
                raise IRBridgeError(f"indirect index must select one element (view shape {e.shape})")
            tid = self.c.tensor_ids[id(base)]
            inner = " ".join(self.index_expr(x) for x in e.index_exprs)
            return f"t {tid} {len(base.shape)} {len(e.index_exprs)} {inner}".rstrip()
        if hasattr(e, "name") and not isinstance(e, (int, float)):
            return f"v {enc(str(e.name))}"
        try:
            return f"c {int(e)}"
        except Exception as ex:  # noqa: BLE001
            raise IRBridgeError(f"Unsupported index expr: {e!r}") from ex

    # -- axes -------------------------------------------------------------
    def axis(self, axis: Any, var_name: str) -> str:
        bound = getattr(axis, "extent_view", None)
        if isinstance(bound, Tensor):
            return f"dynt {int(axis.size)} " + self.index_expr(bound)
        if isinstance(axis, DenseDyn):
            return f"dyn {enc(var_name)}"
        if isinstance(axis, Ragged):
            return f"ragged {enc(f'outer_{id(axis)}')} {enc(f'lengths_{id(axis)}')}"
        if isinstance(axis, Sparse):
            raise IRBridgeError("Sparse axes are only valid under P.sel")
        return f"dense {axis_extent(axis)}"

    @staticmethod
    def axis_arg(v: Any) -> str:
        if hasattr(v, "name") and not isinstance(v, (int, float, str)):
            return f"v {enc(str(v.name))}"
        if isinstance(v, str):
            return f"c {fnv1a_64(v)}"
        try:
            return f"c {int(v) & 0xFFFFFFFFFFFFFFFF}"
        except Exception as ex:  # noqa: BLE001
            raise IRBridgeError(f"Unsupported axis binding value: {v!r}") from ex

    @staticmethod
    def scalar_arg(v: Any, dtype: DType) -> str:
        if isinstance(v, Symbol):
            return f"s {enc(v.sym)} {fnv1a_64(v.sym)}"
        if hasattr(v, "name") and not isinstance(v, (int, float, str)):
            return f"v {enc(str(v.name))}"
        if dtype == DType.F32:
            return f"c {struct.unpack('<I', struct.pack('<f', float(v)))[0]}"
        if dtype == DType.I32:
            return f"c {int(v) & 0xFFFFFFFF}"
        if dtype == DType.I64:
            return f"c {int(v) & 0xFFFFFFFFFFFFFFFF}"
        raise IRBridgeError(f"Unsupported scalar dtype for codegen args: {dtype!r}")

    # -- workload tree ----------------------------------------------------
    def node(self, w: Any) -> None:
        if not isinstance(w, Workload):
            raise IRBridgeError(f"workload body must be a Workload (got {type(w).__name__})")
        kind, kw = w._kind, w._kwargs
        if kind == "empty":
            self.emit("empty")
        elif kind in ("parallel_for", "for_each"):
            var = str(kw.get("var_name", "i"))
            self.emit("pfor" if kind == "parallel_for" else "each", enc(var), self.axis(kw.get("axis"), var))
            self.node(self.c.body(w))
        elif kind in ("combine", "sequential"):
            kids = [c for c in (kw.get("workloads", []) or []) if isinstance(c, Workload)]
            self.emit("comb" if kind == "combine" else "seqn", len(kids))
            for c in kids:
                self.node(c)
        elif kind == "task":
            self.task(w)
        elif kind == "select":
            sp = kw.get("sparse")
            self.emit("sel", enc(str(kw.get("var_name", "e"))), enc(f"outer_{id(sp)}"),
                      enc(f"indptr_{id(sp)}"), enc(f"indices_{id(sp)}"))
            self.node(self.c.body(w))
        elif kind == "cond":
            # python/pto_wsp/ir_bridge.py:485-500 of the reference: the predicate
            # must convert to a ScalarExpr; a missing branch is empty.
            self.emit("cond", as_expr(kw.get("predicate")).to_text())
            then_w, else_w = kw.get("then_workload"), kw.get("else_workload")
            self.node(then_w if isinstance(then_w, Workload) else Workload("empty"))
            self.node(else_w if isinstance(else_w, Workload) else Workload("empty"))
        elif kind == "slot_set_u64":
            self.emit("slotset", int(kw.get("slot", 0)) & 0xFFFFFFFF, int(kw.get("value", 0)) & 0xFFFFFFFFFFFFFFFF)
        elif kind == "slot_load_u64":
            # python/pto_wsp/ir_bridge.py:354-375 of the reference.
            t = kw.get("tensor")
            if not isinstance(t, Tensor):
                raise IRBridgeError("slot_load_u64 requires tensor=Tensor view")
            if len(t.shape) < 2:
                raise IRBridgeError(f"slot_load_u64 tensor view must be rank>=2 (got shape={t.shape!r})")
            tid = self.c.tensor_ids[id(t.base)]
            idx = [self.index_expr(e) for e in t.index_exprs]
            self.emit("slotld", int(kw.get("slot", 0)) & 0xFFFFFFFF, tid, len(t.base.shape), len(t.shape), len(idx),
                      *idx, int(kw.get("row", 0)), int(kw.get("col", 0)))
        else:
            raise IRBridgeError(f"workload node kind '{kind}' is not supported by codegen")

    def task(self, w: Workload) -> None:
        kw = w._kwargs
        kernel = kw.get("kernel")
        if kernel is None or not hasattr(kernel, "name"):
            raise IRBridgeError("Task node missing kernel for codegen")
        resources = kw.get("resources", {})
        if not isinstance(resources, dict):
            raise IRBridgeError("Task resources must be dict[param_name -> Tensor] for codegen")
        ir = kernel.trace()
        axis_args = [self.axis_arg(v) for v in kw.get("params", []) or []]
        sig = inspect.signature(kernel.func)
        scalar_args, tensor_args = [], []
        for pname, pval in ir.params:
            if pval.shape is None:
                if pname in resources:
                    sval = resources[pname]
                else:
                    p = sig.parameters.get(pname)
                    if p is None or p.default is inspect.Parameter.empty:
                        raise IRBridgeError(f"Missing scalar arg for param '{pname}' in task {kernel.name}")
                    sval = p.default
                scalar_args.append(self.scalar_arg(sval, pval.dtype))
                continue
            t = resources.get(pname)
            if not isinstance(t, Tensor):
                raise IRBridgeError(f"Missing tensor arg for param '{pname}' in task {kernel.name}")
            tid = self.c.tensor_ids[id(t.base)]
            idx = [self.index_expr(e) for e in t.index_exprs]
            tensor_args.append(
                f"{enc(pname)} {tid} {len(t.base.shape)} {len(t.shape)} {len(idx)} {' '.join(idx)}".rstrip())
        self.emit("task", enc(kernel.name), len(axis_args), *axis_args, len(scalar_args), *scalar_args,
                  len(tensor_args))
        for ta in tensor_args:
            self.emit(" ", ta)

    # -- kernels ----------------------------------------------------------
    def kernel(self, k: Any) -> None:
        opts = getattr(k, "options", {}) or {}
        # 1: a cpp_src body (cpp_body_path reads one), 2: a whole translation unit (cpp_tu_path).
        custom = 1 if opts.get("cpp_src") is not None else 2 if opts.get("cpp_file_src") is not None else 0
        if custom and opts.get("cpp_includes"):
            raise IRBridgeError(f"kernel {k.name}: cpp_includes name host headers; device bodies cannot include them")
        ir = k.trace()
        values: dict[int, Any] = {}
        for _, v in ir.params:
            values[v.id] = v
        for op in ir.ops:
            if op.result is not None:
                values[op.result.id] = op.result
        directions = {p.name: p.direction for p in k._kernel_params}
        src = opts.get("cpp_src") if custom == 1 else opts.get("cpp_file_src")
        self.emit("K", enc(ir.name), len(values), len(ir.params), len(ir.ops), custom,
                  *([enc(str(src))] if custom else []))
        for vid in sorted(values):
            v = values[vid]
            if v.shape is None:
                self.emit("V", vid, dtype_str(v.dtype), "S")
            else:
                r, c = v.shape
                if not isinstance(r, int) or not isinstance(c, int):
                    raise IRBridgeError(f"Kernel value shape must be concrete ints (got {v.shape!r})")
                self.emit("V", vid, dtype_str(v.dtype), "T", r, c)
        for name, v in ir.params:
            self.emit("P", enc(name), v.id, directions.get(name, "in"))
        for op in ir.ops:
            attrs = self.attrs(op.attrs or {})
            res = op.result.id if op.result is not None else -1
            self.emit("O", op.kind.name, res, len(op.operands), *[o.id for o in op.operands], len(attrs), *attrs)

    @staticmethod
    def attrs(attrs: dict) -> list[str]:
        out = []
        for key, v in attrs.items():
            if isinstance(v, bool):
                out.append(f"{enc(key)} b {int(v)}")
            elif isinstance(v, int):
                out.append(f"{enc(key)} i {v}")
            elif isinstance(v, float):
                if not math.isfinite(v):
                    raise IRBridgeError(f"non-finite attr '{key}'")
                out.append(f"{enc(key)} d {v!r}")
            elif isinstance(v, str):
                out.append(f"{enc(key)} s {enc(v)}")
            elif isinstance(v, (list, tuple)):
                if all(isinstance(x, int) and not isinstance(x, bool) for x in v):
                    out.append(f"{enc(key)} I {len(v)} {' '.join(str(x) for x in v)}".rstrip())
                elif all(isinstance(x, str) for x in v):
                    out.append(f"{enc(key)} S {len(v)} {' '.join(enc(x) for x in v)}".rstrip())
                else:
                    raise IRBridgeError(f"Unsupported attr list type for '{key}': {v!r}")
            else:
                raise IRBridgeError(f"Unsupported attr type for '{key}': {type(v)}")
        return out

    # -- schedule ---------------------------------------------------------
    def schedule(self, w: Workload) -> None:
        directives = []
        sched = w._schedule
        if sched.to_dict():
            if sched.dispatch is not None:
                kind = getattr(sched.dispatch, "_kind", "")
                kwargs = getattr(sched.dispatch, "_kwargs", {}) or {}
                directives.append(f"D {kind or 'custom'} {int(kwargs.get('num_aicpus', 0) or 0)} "
                                  + _dispatch_key_text(kind, kwargs))
            tg = w._task_graph_config
            window = getattr(tg, "window", None) if tg is not None else None
            if window is not None:
                mode = getattr(window.mode, "value", str(window.mode)).lower()
                overflow = "abort" if "abort" in mode else ("benchmark" if "bench" in mode else "stall")
                directives.append(f"W {int(window.size)} {enc(str(window.unit))} {overflow}")
            if sched.streams != 1:
                directives.append(f"S {int(sched.streams or 0)} {1 if sched.stream_by is not None else 0}")
            if sched.timing is not None:
                directives.append(f"M {enc(getattr(sched.timing, '_kind', 'custom'))}")
        self.emit("schedule", len(directives))
        for d in directives:
            self.emit(d)


def _dispatch_key_text(kind: str, kwargs: dict) -> str:
    """``1 <expr>`` for a keyed dispatch policy, ``0`` otherwise (the key is
    traced into a ScalarExpr as python/pto_wsp/ir_bridge.py:619-648 of the
    reference does)."""
    fn = kwargs.get("key_fn") if kind in ("affinity", "hash") else kwargs.get("fn") if kind == "dispatch_by" else None
    if kind in ("affinity", "hash", "dispatch_by") and fn is None:
        raise IRBridgeError(f"DispatchPolicy.{kind} missing {'fn' if kind == 'dispatch_by' else 'key_fn'}")
    if fn is None:
        return "0"
    expr = trace_task_fn(fn) if callable(fn) else as_expr(fn)
    return "1 " + expr.to_text()


def workload_to_codegen_ir(workload: Workload, module_name: str = "main") -> CodegenIRBuild:
    """Serialize ``workload`` (and the kernels it calls) into module text."""
    col = _Collector()
    col.collect(workload)
    w = _Writer(col)
    w.emit(MODULE_MAGIC)
    w.emit("name", enc(module_name))
    w.emit("tensors", len(col.tensors))
    for t in col.tensors:
        w.emit("T", dtype_str(t.dtype), len(t.shape), *t.shape)
    w.emit("kernels", len(col.kernels))
    for _, k in sorted(col.kernels.items()):
        w.kernel(k)
    w.emit("workload", enc(workload._name or "unnamed"))
    w.node(workload)
    w.schedule(workload)
    w.emit("end")
    return CodegenIRBuild(module="\n".join(w.lines) + "\n", tensors=list(col.tensors))
