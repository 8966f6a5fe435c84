"""Random kernels (tests/fuzz_programs.py) on the CPU side.

* the oracle against the float64 referee: each stored result within a
  bound of float64 fitting its dtype (fp32 arithmetic, or the f16 / bf16
  store cast), so the oracle is pinned on op combinations, shapes and
  layouts no hand-written case covers;
* the product's cycle model (C++) against the oracle's: equal total_cycles
  and task counts;
* every launch of every program is accepted, emitted and built for gfx950.
"""

import numpy as np
import pytest

import fuzz_programs as FP
import workloads as W
from oracle.runner import run_workload
from pto_wsp.ir_bridge import workload_to_codegen_ir
from pto_wsp.program import Program

SEEDS = range(0, 80)
ORACLE_BOUND = {FP.F32: 1e-4, FP.F16: 2.0 ** -10, FP.BF16: 2.0 ** -7}


@pytest.mark.parametrize("seed", SEEDS)
def test_random_program_oracle_and_cycles(seed):
    from pto_wsp._hip import NativeProgram

    prog = FP.generate(seed)
    arrs = FP.arrays(prog)
    ca = {k: v.copy() for k, v in arrs.items()}
    w = W.rr4(FP.make_workload(prog, ca))
    ref = run_workload(w)
    f64 = FP.evaluate(prog, arrs)
    dts = {p.name: p.dtype for p in prog.params}
    for name, r in f64.items():
        o = FP._f64(ca[name], dts[name])
        err = float(np.max(np.abs(o - r))) / (float(np.max(np.abs(r))) + 1e-30)
        assert err <= ORACLE_BOUND[dts[name]], f"{name}: {err}\n{prog.describe()}"

    w2 = W.rr4(FP.make_workload(prog, {k: v.copy() for k, v in arrs.items()}))
    build = workload_to_codegen_ir(w2, f"fuzz{seed}")
    native = NativeProgram(build.module)
    got = native.cycle_model(build.tensors, Program._infer_axis_sizes(w2), {}, {})
    assert (got.total_cycles, got.task_count) == (ref.total_cycles, ref.task_count), prog.describe()
    for i in range(native.num_launches()):
        assert "__global__" in native.precompile(i)


def test_referee_rejects_a_planted_mistake():
    """The float64 referee catches a wrong op: the oracle run with the op that produces a stored
    value turned into another (add <-> sub) fails compare(), while its own result passes."""
    for seed in SEEDS:
        prog = FP.generate(seed)
        producer = {res: i for i, (_, _, res) in enumerate(prog.ops)}
        i = producer.get(prog.stores[0][1]) if prog.stores else None
        if i is None or prog.ops[i][0] not in ("add", "sub"):
            continue
        x, y = prog.ops[i][1]
        if not isinstance(y, tuple) and x != y and prog.vals[x].kind == prog.vals[y].kind:
            break
    else:
        pytest.fail("no program whose stored value comes from a tile add or sub")
    arrs = FP.arrays(prog)
    good = {k: v.copy() for k, v in arrs.items()}
    run_workload(W.rr4(FP.make_workload(prog, good)))
    ref = FP.evaluate(prog, arrs)
    assert not FP.compare(prog, good, good, ref)

    op, args, res = prog.ops[i]
    prog.ops[i] = ("sub" if op == "add" else "add", args, res)
    bad = {k: v.copy() for k, v in arrs.items()}
    run_workload(W.rr4(FP.make_workload(prog, bad)))
    assert FP.compare(prog, bad, good, ref)
