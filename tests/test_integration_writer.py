"""The reference-side writer (pto-wsp_amd/integration/hip_target.cpp), CPU only.

The writer turns a reference ir::Module (include/pto/wsp/ir/module.hpp) into
the module text that ptowsp_hip_compile reads.  tests/integration/build.py
compiles it against the reference's headers with a tool that builds three
ir::Modules the way the reference's Python bridge would
(python/pto_wsp/ir_bridge.py:112-139); each must print the same text as this
repository's bridge writes for the same workload (the reference IR carries no
parameter direction, which the target does not read).  The entry shim that
build_hip_artifact compiled for each case must export `<module>_main`.
Skipped when the tool was not built (no reference headers).
"""

import os
import subprocess

import pytest

from integration import cases

TOOL = os.path.join(cases.BUILD, "ir_cases")
needs_tool = pytest.mark.skipif(not os.path.exists(TOOL), reason="integration tool not built (reference headers absent)")


def _normalized(text: str) -> list:
    out = []
    for line in text.splitlines():
        tok = line.split()
        if tok and tok[0] == "P" and len(tok) == 4:
            tok[3] = "*"  # parameter direction: not part of the reference IR
        out.append(("  " if line.startswith("  ") else "") + " ".join(tok))
    return out


@needs_tool
@pytest.mark.parametrize("case", cases.CPP_CASES + ("bgemm_f16",))
def test_cpp_writer_matches_python_bridge(case):
    cpp = subprocess.run([TOOL, "write", case], check=True, capture_output=True, text=True).stdout
    if case == "bgemm_f16":
        import numpy as np
        import workloads as W
        from pto_wsp.ir_bridge import workload_to_codegen_ir

        arrs = {"a": np.zeros((1, 64, 64), np.float16), "b": np.zeros((1, 64, 64), np.float16),
                "c": np.zeros((1, 64, 64), np.float32)}
        py = workload_to_codegen_ir(W.rr4(W.bgemm(arrs)), case).module
    else:
        py = cases.python_text(case)
    assert _normalized(cpp) == _normalized(py)


@needs_tool
def test_cpp_written_text_compiles_on_the_target():
    """The C++-written text parses, plans and has the oracle's cycle model."""
    from pto_wsp import _hip

    for case in cases.CPP_CASES:
        text = subprocess.run([TOOL, "write", case], check=True, capture_output=True, text=True).stdout
        prog = _hip.NativeProgram(text)
        assert prog.num_launches() >= 1


@needs_tool
@pytest.mark.parametrize("case", cases.CPP_CASES + ("paged_decode",))
def test_artifact_exports_its_entry(case):
    art = cases.artifact(case)
    assert art is not None, f"artifact of {case} missing; run __graft_entry__.build()"
    so, entry = art
    assert entry == f"{case}_main"
    syms = subprocess.run(["nm", "-D", "--defined-only", so], check=True, capture_output=True, text=True).stdout
    assert f" T {entry}" in syms
    # The artifact embeds the case's current module text.
    src = open(os.path.join(os.path.dirname(so), "hip_entry.c")).read()
    assert "PTOWSP-MODULE 1" in src and f"name {case}" in src
