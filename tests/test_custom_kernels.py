"""cpp_src and cpp_tu_path kernels (the reference's @kernel escape hatches) on CPU.

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


# The reference's own translation-unit kernel (tests/test_npu_codegen_emit.py:155-206: tu_copy,
# a 4x4 copy through the task descriptor), written anew.
TU_COPY = r"""
#include "pto/wsp/codegen/abi/kernel_abi.hpp"
#include "pto/wsp/codegen/abi/ptoisa_bridge.hpp"
#include <cstdint>
#include <cstddef>

extern "C" PTO_WSP_KERNEL_ATTR uint64_t tu_copy(const KernelTaskDesc* task, CSPTContext* cspt) {
  (void)cspt;
  const float* x = (const float*)task->tensor_ptrs[0];
  float* y = (float*)task->tensor_ptrs[1];
  const int64_t xs3 = (int64_t)task->tensor_strides[0], xs4 = (int64_t)task->tensor_strides[1];
  const int64_t ys3 = (int64_t)task->tensor_strides[2], ys4 = (int64_t)task->tensor_strides[3];
  for (int r = 0; r < 4; ++r)
    for (int c = 0; c < 4; ++c) y[r * ys3 + c * ys4] = x[r * xs3 + c * xs4];
  return 0;
}
"""


def tu_copy_workload(x, y, path):
    X, Y = Tensor(data=x, shape=x.shape, dtype=DType.F32), Tensor(data=y, shape=y.shape, dtype=DType.F32)

    @kernel(cpp_tu_path=str(path))
    def tu_copy(x_tile: In[Tile[4, 4, DType.F32]], y_tile: Out[Tile[4, 4, DType.F32]]):
        pass

    @workload
    def wl():
        tu_copy(x_tile=X, y_tile=Y)

    return wl()


def test_oracle_runs_translation_units(tmp_path):
    """cpp_tu_path kernels: the reference's tu_copy copies exactly with 0 cycles, and the probe
    written as a translation unit (helper function, pto::cpu_sim counter) gives the same
    descriptor contents and cycles as the cpp_src probe."""
    p = tmp_path / "tu_copy.cpp"
    p.write_text(TU_COPY)
    x = np.arange(16, dtype=np.float32).reshape(4, 4)
    y = np.zeros((4, 4), np.float32)
    ref = run_workload(tu_copy_workload(x, y, p))
    np.testing.assert_array_equal(y, x)
    assert (ref.total_cycles, ref.task_count) == (0, 1)

    q = tmp_path / "probe.cpp"
    q.write_text(W.PROBE_TU)
    a = probe_arrays()
    ref = run_workload(W.cpp_probe(a, tu_path=str(q)))
    want, cycles = probe_expected(a)
    np.testing.assert_array_equal(a["o"], want)
    assert (ref.total_cycles, ref.task_count) == (cycles, 12)


def test_translation_units_build_for_gfx950(tmp_path):
    from pto_wsp._hip import NativeProgram

    q = tmp_path / "probe.cpp"
    q.write_text(W.PROBE_TU)
    prog = NativeProgram(workload_to_codegen_ir(W.cpp_probe(probe_arrays(), tu_path=str(q)), "c").module)
    src = prog.precompile(0)
    assert src.startswith("// ptowsp: cpp_tu") and "probe(&d, nullptr)" in src
    assert prog.kernel_family("probe") == "custom"


def test_translation_unit_without_its_entry_or_with_tile_api_is_a_compile_error(tmp_path):
    """A file that does not define extern "C" <kernel name>, or calls PTO-ISA's tile API (absent
    on this backend), fails to build with the compiler's message."""
    from pto_wsp._hip import NativeProgram

    x, y = np.zeros((4, 4), np.float32), np.zeros((4, 4), np.float32)
    for text in (TU_COPY.replace("tu_copy(", "other_name("),
                 TU_COPY.replace("return 0;", "pto_wsp::ptoisa::TADD(y, x, x);\n  return 0;")):
        p = tmp_path / "bad.cpp"
        p.write_text(text)
        prog = NativeProgram(workload_to_codegen_ir(tu_copy_workload(x, y, p), "c").module)
        with pytest.raises(RuntimeError, match="hiprtc failed"):
            prog.precompile(0)


def test_includes_are_refused(tmp_path):
    X = Tensor(data=np.zeros((1, 1, 1, 4), np.float32), shape=(1, 1, 1, 4), dtype=DType.F32)

    @kernel(cpp_src="cycles = 1;", cpp_includes=["pto/pto.hpp"])
    def k_inc(x: In[Tile[1, 4, DType.F32]], y: Out[Tile[1, 4, DType.F32]]):
        pass

    @workload
    def wl():
        for b in P(W.Dense[1]()):
            k_inc[b](x=X[b][0], y=X[b][0])

    with pytest.raises(IRBridgeError, match="cpp_includes"):
        workload_to_codegen_ir(wl())
