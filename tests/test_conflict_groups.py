"""Launches whose grid tasks write overlapping memory (CPU: oracle and emitted code).

P() promises independent iterations; a workload that breaks the promise still
gets the reference's result, which is that of program order.  The oracle runs
every task in program order and is pinned here against float32 sums in that
order; the HIP backend runs such a launch as parallel groups of tasks that
write disjoint memory, each group in program order (its GPU parity is in
tests/test_gpu_conflict_groups.py).
"""

import numpy as np

import workloads as W
from oracle.runner import run_workload


def _arrays(shape, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32) * np.float32(1e3)
    B, S, V, R, C = shape
    return {"x": x, "out": rng.standard_normal((B, V, R, C)).astype(np.float32)}


def test_oracle_sums_overlapping_writes_in_program_order():
    a = _arrays((2, 5, 3, 4, 16), 0)
    want = W.conflict_accumulate_ref(a["x"], a["out"])
    run_workload(W.rr4(W.conflict_accumulate(a)))
    np.testing.assert_array_equal(a["out"], want)
    # another order of the s terms gives other float32 sums
    b = _arrays((2, 5, 3, 4, 16), 0)
    rev = b["out"].copy()
    for s in reversed(range(5)):
        rev = rev + b["x"][:, s]
    assert not np.array_equal(rev, want)


def test_oracle_one_shared_tile():
    a = _arrays((2, 3, 2, 4, 16), 1)
    want = W.conflict_accumulate_ref(a["x"], a["out"], shared_all=True)
    run_workload(W.rr4(W.conflict_accumulate(a, shared_all=True)))
    np.testing.assert_array_equal(a["out"], want)


def test_grouped_variant_builds_for_gfx950():
    from pto_wsp._hip import NativeProgram
    from pto_wsp.ir_bridge import workload_to_codegen_ir

    a = _arrays((2, 5, 3, 4, 16), 0)
    prog = NativeProgram(workload_to_codegen_ir(W.conflict_accumulate(a), "conflict").module)
    src = prog.precompile(0, serial=True, seq_mask=0b010)
    assert "ngroups_ *= A.ext[0];" in src and "ngroups_ *= A.ext[2];" in src
    assert "for (vars[1] = 0; vars[1] < e0; ++vars[1])" in src
