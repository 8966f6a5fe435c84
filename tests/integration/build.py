"""Builds the reference-side integration test support (test infrastructure).

Compiles, with g++ against the reference's headers under /root/reference/include
(C++20, as the reference builds):
  * ir_cases: the reference-side writer (pto-wsp_amd/integration/hip_target.cpp)
    driven on reference ir::Modules, and its artifact builder;
  * abi_main_driver: a foreign loader over the reference's workload_abi.hpp;
then builds the hip_gfx950 artifact of every case in tests/integration/cases.py
with build_hip_artifact, against libptowsp_hip.so (which must be built first).
Outputs go to tests/integration/_build/.  Without the reference headers nothing
is built and the tests that need these files skip.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_INCLUDE = "/root/reference/include"
BUILD = os.path.join(HERE, "_build")


def build() -> bool:
    if not os.path.isdir(os.path.join(REF_INCLUDE, "pto", "wsp", "ir")):
        print("integration: reference headers absent; reference-side integration test support not built", file=sys.stderr)
        return False
    for p in (os.path.join(ROOT, "pto-wsp_amd"), ROOT, os.path.join(ROOT, "tests"), HERE):
        if p not in sys.path:
            sys.path.insert(0, p)
    import cases

    os.makedirs(cases.ARTIFACTS, exist_ok=True)
    integ = os.path.join(ROOT, "pto-wsp_amd", "integration")
    tool = os.path.join(BUILD, "ir_cases")
    driver = os.path.join(BUILD, "abi_main_driver")
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-I", REF_INCLUDE, "-I", integ,
                    os.path.join(HERE, "ir_cases.cpp"), os.path.join(integ, "hip_target.cpp"), "-o", tool], check=True)
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-I", REF_INCLUDE,
                    os.path.join(HERE, "abi_main_driver.cpp"), "-o", driver, "-ldl"], check=True)
    lib_dir = os.path.join(ROOT, "pto-wsp_amd", "pto_wsp")
    include_dir = os.path.join(ROOT, "include")
    for case in (*cases.CPP_CASES, "paged_decode"):
        if case in cases.CPP_CASES:
            text = subprocess.run([tool, "write", case], check=True, capture_output=True, text=True).stdout
        else:
            text = cases.python_text(case)
        mod = os.path.join(BUILD, f"{case}.module")
        with open(mod, "w") as f:
            f.write(text)
        out = subprocess.run([tool, "build", mod, case, cases.ARTIFACTS, include_dir, lib_dir], check=True,
                             capture_output=True, text=True).stdout.split()
        with open(os.path.join(BUILD, f"{case}.artifact"), "w") as f:
            f.write(f"{out[0]} {out[1]}\n")
    return True


if __name__ == "__main__":
    build()
