"""Cases of the reference-side integration test (test support, not product code).

Each case is a module whose hip_gfx950 artifact is built ahead of time by
tests/integration/build.py and run on the GPU by tests/test_gpu_abi_main.py
through a foreign loader (abi_main_driver).  "quickstart" and "slot_branch"
are written by the reference-side C++ writer from a reference ir::Module
(ir_cases write); "paged_decode" uses an indirect page-table index and a
tensor-bound page count, which the reference IR cannot express, so its text
comes from this repository's Python bridge.
"""

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BUILD = os.path.join(HERE, "_build")
ARTIFACTS = os.path.join(BUILD, "artifacts")
CPP_CASES = ("quickstart", "slot_branch")
DECODE_LENGTHS = [37, 16, 1, 100, 64, 5]


def quickstart_workload(arrs):
    import workloads as W

    return W.rr4(W.rmsnorm(arrs))


def slot_branch_workload(arrs):
    import workloads as W

    return W.slot_branch(arrs)


def decode_arrays():
    import workloads as W

    return W.paged_decode_arrays(DECODE_LENGTHS, hkv=2, group=4, d=64, seed=21)


def decode_workload(arrs):
    import workloads as W

    return W.rr4(W.paged_decode(arrs))


def python_text(case: str) -> str:
    """Module text of a case from the Python bridge (for the decode case, the artifact's text)."""
    from pto_wsp.ir_bridge import workload_to_codegen_ir

    if case == "quickstart":
        x = np.zeros((1, 2, 16, 128), np.float32)
        w = quickstart_workload({"x": x, "y": x.copy()})
    elif case == "slot_branch":
        w = slot_branch_workload({k: np.zeros((1, 1, 1, 1), np.int32) for k in ("src", "flag", "y")})
    elif case == "paged_decode":
        w = decode_workload(decode_arrays())
    else:
        raise ValueError(case)
    return workload_to_codegen_ir(w, case).module


def artifact(case: str):
    """(so_path, entrypoint) recorded by the build, or None."""
    rec = os.path.join(BUILD, f"{case}.artifact")
    if not os.path.exists(rec):
        return None
    so, entry = open(rec).read().split()[:2]
    return (so, entry) if os.path.exists(so) else None
