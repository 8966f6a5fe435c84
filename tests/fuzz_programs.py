"""Seeded random kernels for differential tests of the lowering.

A program is a random dataflow over the ops the lowering accepts: tile
binary ops in their same-shape, row-broadcast ([R,1] and [1,R]),
column-broadcast ([1,C] and [C,1]) and scalar forms, exp, rsqrt, the row
reductions, f32 matmul against a per-batch weight tile, and stores with the
f16 / bf16 cast.  Its tiles have random shapes and its tensors random
layouts (a tile may be a transposed view).  It is dispatched either over a
parallel (b, t) grid, optionally updating an InOut tile in place, or with a
P.seq loop over t that folds into InOut accumulators held per b (running
sum or max of a row value, running sum of a full tile), with per-iteration
outputs beside them.

One description is built two ways: as a traced @kernel workload (which the
HIP target and the oracle both run) and as a float64 numpy evaluation, the
referee.  A HIP result passes when it is as close to float64 as the
oracle's own fp32 result is, up to a factor of 4 and a floor, so that a
different summation order passes and a wrong operand, index or op does not.

Values stay where every op is well defined: interval bounds are carried
through the dataflow, so exp sees arguments in [-60, 15], rsqrt and the
divisor of a division stay at least 0.25 away from zero, and magnitudes stay
below 1e4.
"""

from __future__ import annotations

import inspect
import math
from dataclasses import dataclass, field

import numpy as np

import workloads as W
from pto_wsp import DType, Dense, In, InOut, Out, P, Tile, kernel, pto, workload

F32, F16, BF16 = DType.F32, DType.F16, DType.BF16
CONSTS = (-2.5, -1.0, 0.5, 1.5, 3.0)
BOUND = 1e4
BIN = ("add", "sub", "mul", "div", "max", "min")


@dataclass
class Val:
    kind: str   # "full" [R,C], "row" [R,1], "rowT" [1,R], "col" [1,C], "colT" [C,1], "mat" [C,C]
    lo: float
    hi: float


@dataclass
class Param:
    name: str
    kind: str          # as Val.kind
    role: str          # "in", "inout", "out"
    moving: bool       # indexed [b][t] (else [b])
    transposed: bool   # the tile is a transposed view of its array
    dtype: DType = F32
    value: int = -1    # the value id the param provides (inputs)


@dataclass
class Program:
    seed: int
    R: int
    C: int
    B: int
    NT: int
    seq: bool
    params: list = field(default_factory=list)
    vals: list = field(default_factory=list)
    ops: list = field(default_factory=list)      # (op, (operand ids | ("c", const)), result id)
    stores: list = field(default_factory=list)   # (param name, value id)
    acc_ops: dict = field(default_factory=dict)  # accumulator param -> (op, value id) of its update

    def shape(self, kind: str) -> tuple:
        R, C = self.R, self.C
        return {"full": (R, C), "row": (R, 1), "rowT": (1, R), "col": (1, C), "colT": (C, 1), "mat": (C, C)}[kind]

    def describe(self) -> str:
        lines = [f"seed={self.seed} R={self.R} C={self.C} B={self.B} NT={self.NT} seq={self.seq}"]
        for p in self.params:
            lines.append(f"  param {p.name}: {p.role} {p.kind} {p.dtype.name} moving={p.moving} transposed={p.transposed}")
        for op, args, r in self.ops:
            lines.append(f"  v{r} = {op}{args}")
        for name, v in self.stores:
            lines.append(f"  store {name} <- v{v}")
        return "\n".join(lines)


def _interval(op: str, a: Val, b) -> tuple | None:
    """Bounds of op(a, b) for b a Val or a constant, or None when the op is not well defined there."""
    blo, bhi = (b, b) if isinstance(b, float) else (b.lo, b.hi)
    if op == "add":
        lo, hi = a.lo + blo, a.hi + bhi
    elif op == "sub":
        lo, hi = a.lo - bhi, a.hi - blo
    elif op == "mul":
        ps = (a.lo * blo, a.lo * bhi, a.hi * blo, a.hi * bhi)
        lo, hi = min(ps), max(ps)
    elif op == "div":
        if not (blo >= 0.25 or bhi <= -0.25):
            return None
        ps = (a.lo / blo, a.lo / bhi, a.hi / blo, a.hi / bhi)
        lo, hi = min(ps), max(ps)
    elif op == "max":
        lo, hi = max(a.lo, blo), max(a.hi, bhi)
    else:
        lo, hi = min(a.lo, blo), min(a.hi, bhi)
    if max(abs(lo), abs(hi)) > BOUND:
        return None
    return lo, hi


def generate(seed: int) -> Program:
    rng = np.random.default_rng(seed)
    R = int(rng.choice([1, 2, 3, 4, 5, 8, 16, 32]))
    C = int(rng.choice([8, 12, 16, 24, 32, 40, 64, 96, 128, 256, 512]))
    if R * C > 16384:
        R = max(1, 16384 // C)
    B, NT = int(rng.integers(1, 4)), int(rng.integers(1, 6))
    if rng.random() < 0.2:  # a grid larger than one row program's tasks per workgroup
        B, NT = int(rng.integers(2, 6)), int(rng.integers(8, 40))
    prog = Program(seed, R, C, B, NT, bool(rng.random() < 0.45))

    def add_input(kind, moving=True, transposed=False, lo=-2.0, hi=2.0):
        prog.vals.append(Val(kind, lo, hi))
        p = Param(f"p{len(prog.params)}", kind, "in", moving, transposed, F32, len(prog.vals) - 1)
        prog.params.append(p)
        return p

    for _ in range(int(rng.integers(1, 3))):
        add_input("full", transposed=bool(rng.random() < 0.3))
    if rng.random() < 0.5:
        add_input(str(rng.choice(["row", "rowT"])))
    if rng.random() < 0.4:
        add_input(str(rng.choice(["col", "colT"])))
    if prog.seq and rng.random() < 0.5:
        add_input("row", moving=False)  # a fixed per-b input, like a running max read by a later phase
    if rng.random() < 0.15 and C <= 128:
        add_input("mat", moving=False, lo=-1.0, hi=1.0)
    inout = None
    if not prog.seq and rng.random() < 0.3:
        inout = prog.params[0]
        inout.role = "inout"

    def of_kind(*kinds):
        return [i for i, v in enumerate(prog.vals) if v.kind in kinds]

    def emit(op, args, kind, lo, hi):
        prog.vals.append(Val(kind, lo, hi))
        prog.ops.append((op, args, len(prog.vals) - 1))

    def try_op() -> bool:
        form = str(rng.choice(["same", "same", "rowb", "colb", "scalar", "exp", "rsqrt", "reduce", "reduce", "matmul"]))
        if form == "same":
            kind = str(rng.choice(["full", "row"]))
            cand = of_kind(kind)
            if not cand:
                return False
            a, b = int(rng.choice(cand)), int(rng.choice(cand))
            op = str(rng.choice(BIN))
            iv = _interval(op, prog.vals[a], prog.vals[b])
            if iv is None:
                return False
            emit(op, (a, b), kind, *iv)
        elif form == "rowb":
            fulls, rows = of_kind("full"), of_kind("row", "rowT")
            if not fulls or not rows:
                return False
            a, b = int(rng.choice(fulls)), int(rng.choice(rows))
            op = str(rng.choice(BIN))
            iv = _interval(op, prog.vals[a], prog.vals[b])
            if iv is None:
                return False
            emit(op, (a, b), "full", *iv)
        elif form == "colb":
            fulls, cols = of_kind("full"), of_kind("col", "colT")
            if not fulls or not cols:
                return False
            a, b = int(rng.choice(fulls)), int(rng.choice(cols))
            op = str(rng.choice(["sub", "mul", "div"]))
            iv = _interval(op, prog.vals[a], prog.vals[b])
            if iv is None:
                return False
            emit(op, (a, b), "full", *iv)
        elif form == "scalar":
            cand = of_kind("full", "row")
            if not cand:
                return False
            a, c = int(rng.choice(cand)), float(rng.choice(CONSTS))
            op = str(rng.choice(BIN))
            iv = _interval(op, prog.vals[a], c)
            if iv is None:
                return False
            emit(op, (a, ("c", c)), prog.vals[a].kind, *iv)
        elif form == "exp":
            cand = [i for i in of_kind("full", "row") if -60.0 <= prog.vals[i].lo and prog.vals[i].hi <= 15.0]
            if not cand:
                return False
            a = int(rng.choice(cand))
            emit("exp", (a,), prog.vals[a].kind, math.exp(prog.vals[a].lo), math.exp(prog.vals[a].hi))
        elif form == "rsqrt":
            cand = [i for i in of_kind("full", "row") if prog.vals[i].lo >= 0.25]
            if not cand:
                return False
            a = int(rng.choice(cand))
            emit("rsqrt", (a,), prog.vals[a].kind, 1.0 / math.sqrt(prog.vals[a].hi), 1.0 / math.sqrt(prog.vals[a].lo))
        elif form == "reduce":
            cand = of_kind("full")
            if not cand:
                return False
            a = int(rng.choice(cand))
            op = str(rng.choice(["rowsum", "rowmax", "rowmean"]))
            v = prog.vals[a]
            lo, hi = (v.lo * C, v.hi * C) if op == "rowsum" else (v.lo, v.hi)
            if max(abs(lo), abs(hi)) > BOUND:
                return False
            emit(op, (a,), "row", lo, hi)
        else:
            fulls, mats = of_kind("full"), of_kind("mat")
            if not fulls or not mats:
                return False
            a = int(rng.choice(fulls))
            m = max(abs(prog.vals[a].lo), abs(prog.vals[a].hi)) * C
            if m > BOUND:
                return False
            emit("matmul", (a, int(mats[0])), "full", -m, m)
        return True

    n_ops = int(rng.integers(1, 8))
    done = 0
    for _ in range(200):
        if done == n_ops:
            break
        done += bool(try_op())

    # Results: the last full value always, and often a row value.
    fulls = of_kind("full")
    last_full = fulls[-1]
    rows = of_kind("row")

    def add_out(kind, value, moving=True, role="out", transposed=False, dtype=F32):
        p = Param(f"p{len(prog.params)}", kind, role, moving, transposed, dtype)
        prog.params.append(p)
        prog.stores.append((p.name, value))
        return p

    if not prog.seq:
        if inout is not None and rng.random() < 0.7:
            prog.stores.append((inout.name, last_full))
        else:
            dt = F32 if rng.random() < 0.6 else (F16 if rng.random() < 0.5 else BF16)
            add_out("full", last_full, transposed=bool(rng.random() < 0.25), dtype=dt)
        if rows and rng.random() < 0.5:
            add_out("row", int(rows[-1]))
    else:
        made = False
        if rows and rng.random() < 0.7:
            r = int(rows[-1])
            op = str(rng.choice(["add", "max"]))
            p = Param(f"p{len(prog.params)}", "row", "inout", False, False, F32)
            prog.params.append(p)
            prog.acc_ops[p.name] = (op, r)
            made = True
        if rng.random() < 0.4 or not made:
            v = prog.vals[last_full]
            if max(abs(v.lo), abs(v.hi)) * prog.NT <= BOUND and rng.random() < 0.5:
                p = Param(f"p{len(prog.params)}", "full", "inout", False, False, F32)
                prog.params.append(p)
                prog.acc_ops[p.name] = ("add", last_full)
            else:
                add_out("full", last_full, transposed=bool(rng.random() < 0.25))
    return prog


# ---------------------------------------------------------------- arrays
def arrays(prog: Program) -> dict:
    """Seeded host arrays of every param, in the layout the views read."""
    rng = np.random.default_rng(prog.seed + 1_000_003)
    out = {}
    for p in prog.params:
        r, c = prog.shape(p.kind)
        lead = (prog.B, prog.NT) if p.moving else (prog.B,)
        shp = lead + ((c, r) if p.transposed else (r, c))
        if p.role == "out":
            np_dt = {F32: np.float32, F16: np.float16, BF16: np.uint16}[p.dtype]
            out[p.name] = np.zeros(shp, np_dt)
        elif p.kind == "mat":
            out[p.name] = rng.uniform(-1.0, 1.0, shp).astype(np.float32)
        else:
            out[p.name] = rng.uniform(-2.0, 2.0, shp).astype(np.float32)
    return out


def _view(arr, transposed: bool):
    if not transposed:
        return arr
    nd = arr.ndim
    axes = tuple(range(nd - 2)) + (nd - 1, nd - 2)
    return arr.permute(*axes) if hasattr(arr, "permute") else arr.transpose(*axes)


# ---------------------------------------------------------------- traced workload
def make_workload(prog: Program, arrs: dict):
    """The program as a @kernel + @workload over arrs (numpy arrays or device tensors)."""
    direction = {"in": In, "inout": InOut, "out": Out}
    annotations = {}
    for p in prog.params:
        r, c = prog.shape(p.kind)
        annotations[p.name] = direction[p.role][Tile[r, c, p.dtype]]

    def body(**kw):
        vals = [None] * len(prog.vals)
        for p in prog.params:
            if p.value >= 0:
                vals[p.value] = kw[p.name]
        for op, args, res in prog.ops:
            xs = [pto.constant(a[1], F32) if isinstance(a, tuple) else vals[a] for a in args]
            fn = {"max": pto.max, "min": pto.min}.get(op) or getattr(pto, op)
            vals[res] = fn(*xs)
        for name, (op, v) in prog.acc_ops.items():
            pto.store(kw[name], getattr(pto, op)(kw[name], vals[v]))
        for name, v in prog.stores:
            pto.store(kw[name], vals[v])

    body.__signature__ = inspect.Signature(
        [inspect.Parameter(p.name, inspect.Parameter.KEYWORD_ONLY) for p in prog.params])
    body.__annotations__ = annotations
    body.__name__ = body.__qualname__ = f"fuzz_{prog.seed}"
    kern = kernel(body)

    tensors = {p.name: W.T(_view(arrs[p.name], p.transposed), p.dtype) for p in prog.params}
    bb, tt = Dense[prog.B](), Dense[prog.NT]()
    loop_t = P.seq if prog.seq else P

    @workload
    def fuzz_wl():
        for b in P(bb):
            for t in loop_t(tt):
                kern[b, t](**{p.name: (tensors[p.name][b][t] if p.moving else tensors[p.name][b]) for p in prog.params})

    fuzz_wl.__name__ = f"fuzz_wl_{prog.seed}"
    return fuzz_wl()


# ---------------------------------------------------------------- float64 referee
def _f64(arr, dtype: DType) -> np.ndarray:
    if dtype == BF16:
        return (arr.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return np.asarray(arr).astype(np.float64)


def evaluate(prog: Program, arrs: dict) -> dict:
    """Float64 results of every stored param, in its array's layout."""
    R, C = prog.R, prog.C
    state = {p.name: _f64(arrs[p.name], p.dtype).copy() for p in prog.params}

    def tile(p, b, t):
        a = state[p.name][b, t] if p.moving else state[p.name][b]
        return a.T if p.transposed else a

    def put(p, b, t, v):
        v = v.T if p.transposed else v
        if p.moving:
            state[p.name][b, t] = v
        else:
            state[p.name][b] = v

    def bcast(v, kind):
        if kind == "rowT":
            return v.reshape(R, 1)
        if kind == "colT":
            return v.reshape(1, C)
        return v

    for b in range(prog.B):
        for t in range(prog.NT):
            vals = [None] * len(prog.vals)
            for p in prog.params:
                if p.value >= 0:
                    vals[p.value] = tile(p, b, t).copy()
            for op, args, res in prog.ops:
                if op in BIN:
                    x = vals[args[0]]
                    y = args[1][1] if isinstance(args[1], tuple) else bcast(vals[args[1]], prog.vals[args[1]].kind)
                    if prog.vals[args[0]].kind == "row" and not isinstance(args[1], tuple):
                        y = y.reshape(R, 1)
                    vals[res] = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide,
                                 "max": np.maximum, "min": np.minimum}[op](x, y)
                elif op == "exp":
                    vals[res] = np.exp(vals[args[0]])
                elif op == "rsqrt":
                    vals[res] = 1.0 / np.sqrt(vals[args[0]])
                elif op == "rowsum":
                    vals[res] = vals[args[0]].sum(axis=1, keepdims=True)
                elif op == "rowmax":
                    vals[res] = vals[args[0]].max(axis=1, keepdims=True)
                elif op == "rowmean":
                    vals[res] = vals[args[0]].mean(axis=1, keepdims=True)
                elif op == "matmul":
                    vals[res] = vals[args[0]] @ vals[args[1]]
                else:
                    raise AssertionError(op)
            by_name = {p.name: p for p in prog.params}
            for name, (op, v) in prog.acc_ops.items():
                p = by_name[name]
                cur = tile(p, b, t)
                put(p, b, t, np.add(cur, vals[v]) if op == "add" else np.maximum(cur, vals[v]))
            for name, v in prog.stores:
                put(by_name[name], b, t, vals[v])
    return {name: state[name] for name in _stored(prog)}


def _stored(prog: Program) -> list:
    return sorted({n for n, _ in prog.stores} | set(prog.acc_ops))


# ---------------------------------------------------------------- the check
FLOOR = {F32: 1e-5, F16: 2.0 ** -10, BF16: 2.0 ** -7}


def compare(prog: Program, got: dict, oracle: dict, ref: dict) -> list:
    """Failures (text) of got against ref, judged by the oracle's own error."""
    dts = {p.name: p.dtype for p in prog.params}
    bad = []
    for name in _stored(prog):
        r = ref[name]
        g, o = _f64(got[name], dts[name]), _f64(oracle[name], dts[name])
        scale = float(np.max(np.abs(r))) + 1e-30
        e_o = float(np.max(np.abs(o - r))) / scale
        e_g = float(np.max(np.abs(g - r))) / scale if np.all(np.isfinite(g)) else math.inf
        if not e_g <= 4.0 * e_o + FLOOR[dts[name]]:
            bad.append(f"{name}: error vs float64 {e_g:.3g} (oracle {e_o:.3g}, scale {scale:.3g})")
    return bad
