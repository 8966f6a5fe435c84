"""cpp_src kernels (the reference's @kernel(cpp_src=...) escape hatch) on CPU.

The oracle runs each body compiled with g++ inside the reference's wrapper
(src/python/pto_codegen.cpp:3294-3324) and must give the known answers:
the branch outcomes of tests/test_codegen_slots_tensor_predicate.py (bodies
written anew here), and, for a probe body that copies its task descriptor
into its output, the descriptor layout the reference defines: args = axis
args, (rows, cols) per tile param, scalar args (src/python/pto_codegen.cpp:
2503-2545); num_axis_args counts the (rows, cols) pairs; tensor strides are
(s3, s4) pairs in elements.  On the HIP side the same bodies must build for
gfx950 (hiprtc); what they compute is compared on the GPU.
"""

import os

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from pto_wsp import DType, In, IRBridgeError, Out, P, Tensor, Tile, kernel, workload, CompileError
from pto_wsp.ir_bridge import workload_to_codegen_ir
from pto_wsp.program import Program


def slot_arrays(x):
    return {"x": np.full((1, 1, 1, 1), x, np.float32), "flag": np.full((1, 1, 1, 1), 9, np.int32),
            "y": np.zeros((1, 1, 1, 1), np.int32)}


@pytest.mark.parametrize("x,flag,y", [(-1.0, 0, 3), (1.0, 1, 7), (0.0, 0, 3)])
def test_oracle_runs_cpp_src_bodies(x, flag, y):
    a = slot_arrays(x)
    ref = run_workload(W.cpp_slot_branch(a))
    assert (int(a["flag"].item()), int(a["y"].item())) == (flag, y)
    assert (ref.total_cycles, ref.task_count) == (2, 2)  # one cycle per body, two tasks in sequence


def probe_arrays(nb=3, nh=2, ni=2):
    x = np.arange(nb * nh * 8, dtype=np.float32).reshape(nb, nh, 2, 4)
    return {"x": x, "o": np.full((ni, nb, nh, 2, 16), -1.0, np.float32)}


def probe_expected(a, keep=lambda b, h: True):
    x, o = a["x"], np.full_like(a["o"], -1.0)
    ni, nb, nh = o.shape[:3]
    s_bits = np.frombuffer(np.float32(2.5).tobytes(), np.uint32)[0]
    cycles = 0
    for i in range(ni):
        for b in range(nb):
            for h in range(nh):
                if not keep(b, h):
                    continue
                args = [b, h, i, 2, 4, 2, 16, int(s_bits)]
                o[i, b, h, 0, :len(args)] = np.asarray(args, np.uint64).astype(np.float32)
                o[i, b, h, 1, :5] = [7, 2, 4, 1, x[b, h, 0, 0] + x[b, h, 1, 0]]
                cycles += 5 + 3 * b + h + 100 * i
    return o, cycles


def test_oracle_task_descriptor_layout():
    a = probe_arrays()
    ref = run_workload(W.cpp_probe(a))
    want, cycles = probe_expected(a)
    np.testing.assert_array_equal(a["o"], want)
    assert (ref.total_cycles, ref.task_count) == (cycles, 12)


def test_oracle_masked_cpp_src_tasks():
    from pto_wsp.scalar_expr import axis

    a = probe_arrays()
    ref = run_workload(W.cpp_probe(a, axis("b") != 1))
    want, cycles = probe_expected(a, lambda b, h: b != 1)
    np.testing.assert_array_equal(a["o"], want)
    assert (ref.total_cycles, ref.task_count) == (cycles, 8)


def test_cpp_src_bodies_build_for_gfx950():
    from pto_wsp._hip import NativeProgram

    for w in (W.cpp_slot_branch(slot_arrays(1.0)), W.cpp_probe(probe_arrays())):
        prog = NativeProgram(workload_to_codegen_ir(w, "c").module)
        for i in range(prog.num_launches()):
            src = prog.precompile(i)
            assert "ptowsp_body" in src and "KernelTaskDesc" in src
    assert NativeProgram(workload_to_codegen_ir(W.cpp_probe(probe_arrays()), "c").module).kernel_family("probe") == "custom"


def test_cycle_model_of_cpp_src_needs_a_run():
    from pto_wsp._hip import NativeProgram

    w = W.cpp_probe(probe_arrays())
    build = workload_to_codegen_ir(w, "c")
    with pytest.raises(RuntimeError, match="known only after it runs"):
        NativeProgram(build.module).cycle_model(build.tensors, {}, {}, {})


def test_translation_units_and_includes_are_refused(tmp_path):
    tu = tmp_path / "k.cpp"
    tu.write_text('extern "C" uint64_t k(const KernelTaskDesc*, CSPTContext*) { return 1; }\n')
    X = Tensor(data=np.zeros((1, 1, 1, 4), np.float32), shape=(1, 1, 1, 4), dtype=DType.F32)

    def wl_of(kern):
        @workload
        def wl():
            for b in P(W.Dense[1]()):
                kern[b](x=X[b][0], y=X[b][0])

        return wl()

    @kernel(cpp_tu_path=str(tu))
    def k_tu(x: In[Tile[1, 4, DType.F32]], y: Out[Tile[1, 4, DType.F32]]):
        pass

    with pytest.raises(CompileError, match="translation unit"):
        Program(wl_of(k_tu), "hip_gfx950", {})

    @kernel(cpp_src="cycles = 1;", cpp_includes=["pto/pto.hpp"])
    def k_inc(x: In[Tile[1, 4, DType.F32]], y: Out[Tile[1, 4, DType.F32]]):
        pass

    with pytest.raises(IRBridgeError, match="cpp_includes"):
        workload_to_codegen_ir(wl_of(k_inc))
    assert os.path.exists(str(tu))
