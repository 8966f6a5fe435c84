"""The drop-in route end to end on the GPU: `<module>_main(RuntimeContext*, CSPTContext*)`.

Each case's artifact (the entry shim that the reference-side
build_hip_artifact wrote and compiled, embedding the module text; see
tests/integration/build.py) is loaded by abi_main_driver, a loader built
against the reference's workload_abi.hpp whose RuntimeContext callbacks are its
own (host buffers, axis sizes, symbols, 256 zeroed slots), as the reference's
CodegenRuntime provides them (src/python/pto_codegen.cpp:3453-3508).  The
outputs it writes back and the total_cycles it returns must equal the CPU
oracle's on the same inputs.  The driver runs as a child process.
"""

import os
import subprocess

import numpy as np
import pytest

import workloads as W
from integration import cases
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(cases.BUILD, "abi_main_driver")


def _run(case, tensors, tmp_path, extra=()):
    """tensors: list of (tid, numpy view, base array of that view); returns (total_cycles, the views
    over the written-back buffers by tid, the driver's output)."""
    art = cases.artifact(case)
    if art is None or not os.path.exists(DRIVER):
        pytest.skip("integration artifacts not built (reference headers absent at build time)")
    # The artifact must embed the module this test's inputs were made for.
    assert open(os.path.join(cases.BUILD, f"{case}.module")).read().split("\n", 2)[2] == \
        cases.python_text(case).split("\n", 2)[2] or case in cases.CPP_CASES
    lines = []
    files = {}
    for tid, v, base in tensors:
        assert base.flags.c_contiguous and v.ctypes.data == base.ctypes.data
        path = str(tmp_path / f"t{tid}.bin")
        base.tofile(path)
        files[tid] = (path, v, base)
        strides = [s // v.itemsize for s in v.strides]
        lines.append(f"tensor {tid} {v.itemsize} {v.ndim} {' '.join(str(d) for d in v.shape)} "
                     f"{' '.join(str(s) for s in strides)} {path}")
    lines += list(extra)
    man = tmp_path / "manifest.txt"
    man.write_text("\n".join(lines) + "\n")
    print(f"abi main: {case}", flush=True)
    p = subprocess.run([DRIVER, art[0], art[1], str(man)], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    out = p.stdout.split()
    cycles = int(out[out.index("total_cycles") + 1])
    outs = {}
    for tid, (path, v, base) in files.items():
        buf = np.fromfile(path + ".out", dtype=base.dtype).reshape(base.shape)
        outs[tid] = np.lib.stride_tricks.as_strided(buf, shape=v.shape, strides=v.strides)
    return cycles, outs, p.stdout


def test_quickstart_through_module_main(gpu, tmp_path):
    x = np.random.default_rng(31).standard_normal((1, 2, 16, 128), dtype=np.float32)
    y = np.zeros_like(x)
    cycles, outs, _ = _run("quickstart", [(0, x, x), (1, y, y)], tmp_path)
    ref = {"x": x.copy(), "y": np.zeros_like(x)}
    r = run_workload(cases.quickstart_workload(ref))
    np.testing.assert_allclose(outs[1], ref["y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(outs[0], x)
    assert cycles == r.total_cycles == 8240


@pytest.mark.parametrize("value,want", [(5, 7), (0, 3)])
def test_slot_branch_through_module_main(gpu, tmp_path, value, want):
    """The foreign context's slot callbacks carry the slot the run loads and the branch it picks."""
    src = np.full((1, 1, 1, 1), value, np.int32)
    zero = np.zeros((1, 1, 1, 1), np.int32)
    cycles, outs, stdout = _run("slot_branch", [(0, src, src), (1, zero, zero), (2, zero, zero)], tmp_path)
    ref = {"src": src.copy(), "flag": zero.copy(), "y": zero.copy()}
    r = run_workload(cases.slot_branch_workload(ref))
    assert outs[2].item() == want == ref["y"].item()
    assert outs[1].item() == value
    assert cycles == r.total_cycles
    assert (f"slot 0 {value}" in stdout) == (value != 0)


def test_paged_decode_through_module_main(gpu, tmp_path):
    a = cases.decode_arrays()
    # Tensor ids in the bridge's first-use order (the page counts bound the page loop first);
    # K is read through its transposed view.
    kt = a["k_cache"].transpose(0, 1, 3, 2)
    order = ["npages", "q", "k_t", "page_table", "v_cache", "mask", "m", "l", "o", "out"]
    views = {k: (a[k], a[k]) for k in order if k != "k_t"}
    views["k_t"] = (kt, a["k_cache"])
    text = open(os.path.join(cases.BUILD, "paged_decode.module")).read().splitlines()
    shapes = [tuple(int(v) for v in l.split()[3:]) for l in text if l.startswith("T ")]
    assert shapes == [tuple(views[k][0].shape) for k in order]
    cycles, outs, _ = _run("paged_decode", [(i, *views[k]) for i, k in enumerate(order)], tmp_path)
    ref = {k: v.copy() for k, v in a.items()}
    r = run_workload(cases.decode_workload(ref))
    got = outs[order.index("out")]
    rel = np.linalg.norm(got - ref["out"]) / np.linalg.norm(ref["out"])
    assert rel <= 1e-5, rel
    want = W.paged_decode_ref(a)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-2
    assert cycles == r.total_cycles
