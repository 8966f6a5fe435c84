"""cond (P.when / P.otherwise / primitives.cond), run-time slots and keyed dispatch (CPU).

* The oracle reproduces the known answers of the reference's own tests:
  tests/test_codegen_cond.py (both predicates), the cycle counts of
  tests/test_codegen_scalar_expr_eval.py (6, 3, 5 and 6 tasks' worth on the
  busiest lane), and the branch outcomes of
  tests/test_codegen_slots_tensor_predicate.py (its cpp_src kernels restated
  as compute kernels: a copy writes the flag, fills write 7 / 3).
* The product's cycle model (total_cycles, task count) equals the oracle's on
  every one of these workloads and bindings.
* Predicates that read a variable out of scope or a task parameter, and keyed
  dispatch without a key, are refused at compile time as the reference's
  emitter refuses them.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from pto_wsp import CompileError, DispatchPolicy, IRBridgeError, P
from pto_wsp.ir_bridge import workload_to_codegen_ir
from pto_wsp.program import Program
from pto_wsp.scalar_expr import axis, fnv1a_64, symbol_u64, task_param


def cond_arrays():
    return {"a0": np.full((4, 1, 2, 2), 1.0, np.float32), "a1": np.full((4, 1, 2, 2), 2.0, np.float32),
            "c": np.zeros((4, 1, 2, 2), np.float32)}


def product_cycles(make, arrs, symbols_u64=None, name="main"):
    from pto_wsp._hip import NativeProgram

    w = make(arrs)
    build = workload_to_codegen_ir(w, name)
    return NativeProgram(build.module).cycle_model(build.tensors, Program._infer_axis_sizes(w), symbols_u64 or {}, {})


def check_product(make, arrs_fn, symbols_u64=None):
    """Oracle and product cycle model on fresh copies of the same arrays."""
    ref = run_workload(make(arrs_fn()), symbols_u64=symbols_u64)
    got = product_cycles(make, arrs_fn(), symbols_u64)
    assert (got.total_cycles, got.task_count) == (ref.total_cycles, ref.task_count)
    return ref


# ---------------------------------------------------------------- reference known answers
def test_cond_runtime_predicate_by_axis_var():
    a = cond_arrays()
    run_workload(W.cond_copy(a, axis("b") < 2))
    np.testing.assert_array_equal(a["c"][:2], a["a0"][:2])
    np.testing.assert_array_equal(a["c"][2:], a["a1"][2:])
    check_product(lambda x: W.cond_copy(x, axis("b") < 2), cond_arrays)


@pytest.mark.parametrize("cut,split", [(2, 2), (1, 1), (0, 0), (9, 4)])
def test_cond_runtime_predicate_by_symbol(cut, split):
    pred = axis("b") < symbol_u64("cut").cast_i64()
    a = cond_arrays()
    syms = {fnv1a_64("cut"): cut}
    run_workload(W.cond_copy(a, pred), symbols_u64=syms)
    np.testing.assert_array_equal(a["c"][:split], a["a0"][:split])
    np.testing.assert_array_equal(a["c"][split:], a["a1"][split:])
    check_product(lambda x: W.cond_copy(x, pred), cond_arrays, syms)


def _copy_arrays():
    a = np.arange(6 * 4 * 4, dtype=np.float32).reshape(6, 4, 4)
    return {"a": a, "b": np.zeros_like(a)}


def _keyed(policy):
    return lambda arrs: W.copy_tiles(arrs, 6).dispatch(policy)


def test_scalar_expr_dispatch_keys():
    serial = run_workload(W.copy_tiles(_copy_arrays(), 6))
    assert serial.total_cycles % 6 == 0
    per = serial.total_cycles // 6
    by_tags = DispatchPolicy.affinity(lambda t: (t.tags["mask"] & t.params[0].cast_u64()), num_aicpus=2)
    ternary = DispatchPolicy.affinity(
        lambda t: (t.params[0] == symbol_u64("special").cast_i64()).where(0, 1).cast_u64(), num_aicpus=2)
    for policy, sym, value, lanes in [(by_tags, "mask", 0, 6), (by_tags, "mask", 1, 3),
                                      (ternary, "special", 0, 5), (ternary, "special", 7, 6)]:
        arrs = _copy_arrays()
        syms = {fnv1a_64(sym): value}
        ref = run_workload(_keyed(policy)(arrs), symbols_u64=syms)
        np.testing.assert_array_equal(arrs["b"], arrs["a"])
        assert ref.total_cycles == lanes * per
        got = product_cycles(_keyed(policy), _copy_arrays(), syms)
        assert (got.total_cycles, got.task_count) == (ref.total_cycles, 6)


def _slot_arrays(src):
    return {"src": np.full((1, 1, 1, 1), src, np.int32), "flag": np.full((1, 1, 1, 1), src, np.int32),
            "y": np.zeros((1, 1, 1, 1), np.int32)}


@pytest.mark.parametrize("src,flag,y", [(-1, -1, 7), (0, 0, 3), (1, 1, 7)])
def test_slot_load_from_tensor_drives_cond(src, flag, y):
    a = _slot_arrays(src)
    a["flag"][:] = 5  # overwritten by the first task before the slot load reads it
    run_workload(W.slot_branch(a))
    assert int(a["flag"].item()) == flag and int(a["y"].item()) == y
    check_product(W.slot_branch, lambda: _slot_arrays(src))


def _chain_arrays():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 4, 8)).astype(np.float32)
    return {"x": x, "y": np.zeros_like(x), "src": np.array([3, 0, 8, 5, 1, 2], np.int32).reshape(6, 1, 1),
            "sel": np.array([3, 0, 8, 5, 1, 2], np.int32).reshape(6, 1, 1)}


def test_slot_loads_inside_a_parallel_loop():
    a = _chain_arrays()
    run_workload(W.slot_chain(a))
    odd = (a["src"].reshape(6) & 1) == 1
    np.testing.assert_allclose(a["y"][odd], a["x"][odd] * 2, rtol=0)
    np.testing.assert_allclose(a["y"][~odd], a["x"][~odd] + 1, rtol=0)
    check_product(W.slot_chain, _chain_arrays)


@pytest.mark.parametrize("pred", [
    lambda: ((axis("b") + axis("t")) % 3) != 0,
    lambda: (axis("t") >= 2) & (axis("b") == 1),
    lambda: ~(axis("t") < symbol_u64("n").cast_i64()),
])
def test_grid_masks_cycle_model(pred):
    def arrs():
        x = np.random.default_rng(1).standard_normal((2, 5, 16, 128)).astype(np.float32)
        return {"x": x, "y": np.zeros_like(x)}

    check_product(lambda a: W.masked_rmsnorm(a, pred()), arrs, {fnv1a_64("n"): 3})


# ---------------------------------------------------------------- refusals
def test_predicate_out_of_scope_is_refused():
    with pytest.raises(CompileError, match="axis_var not in scope"):
        Program(W.cond_copy(cond_arrays(), axis("q") < 2), "hip_gfx950", {})


def test_task_param_in_a_cond_is_refused():
    with pytest.raises(CompileError, match="task_param"):
        Program(W.cond_copy(cond_arrays(), task_param(0) < 2), "hip_gfx950", {})


def test_keyed_dispatch_needs_a_key():
    w = W.copy_tiles(_copy_arrays(), 6).dispatch(DispatchPolicy("custom", num_aicpus=2))
    with pytest.raises(CompileError, match="requires ScalarExpr key"):
        Program(w, "hip_gfx950", {})
    with pytest.raises(IRBridgeError, match="missing key_fn"):
        workload_to_codegen_ir(W.copy_tiles(_copy_arrays(), 6).dispatch(DispatchPolicy("affinity", num_aicpus=2)))


def test_predicate_must_be_a_scalar_expr():
    with pytest.raises(TypeError):
        workload_to_codegen_ir(W.cond_copy(cond_arrays(), "b < 2"))


def test_cond_compiles_for_the_gpu():
    Program(W.cond_copy(cond_arrays(), axis("b") < 2), "hip_gfx950", {})
    Program(W.slot_branch(_slot_arrays(0)), "hip_gfx950", {})
    assert P.when is not None
