"""GPU tests of ptowsp_hip_launch_noalloc, called through the C ABI.

The no-allocation entry point must give the same results as
ptowsp_hip_launch: the paged decode (whose kernels use the scratch buffer:
unit counters and partials) is run through both on the same program and
bindings, twice in a row with a smaller second input, and the outputs must be
identical bit for bit, with identical cycle-model results, and the device's
free memory (hipMemGetInfo) must be the same before and after the
no-allocation run.  Also checked: a decode launch that needs more than the
fixed scratch is refused with an error, and host-resident tensors are
refused.
"""

import ctypes

import numpy as np
import pytest

import workloads as W
from pto_wsp import _hip
from pto_wsp.ir_bridge import workload_to_codegen_ir

pytestmark = pytest.mark.gpu

_lib = _hip.library()
_lib.ptowsp_hip_launch_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.POINTER(_hip.RunInfo)]
_lib.ptowsp_hip_launch_noalloc.restype = ctypes.c_int


class AbiProgram:
    """A compiled module driven through the C ABI entry points directly."""

    def __init__(self, wl, name):
        build = workload_to_codegen_ir(wl, name)
        self.tensors = build.tensors
        self.prog = _hip.NativeProgram(build.module)
        self.live, _ = self.prog._bind(self.tensors, {}, {}, {})
        self.ctx = _lib.ptowsp_rt_context(self.prog._rt)

    def run(self, entry):
        import torch

        stream = torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())
        info = _hip.RunInfo()
        _lib.ptowsp_rt_reset_slots(self.prog._rt)
        if entry(self.prog._h, self.ctx, ctypes.c_void_p(stream), ctypes.byref(info)) != 0:
            raise RuntimeError(_hip._error())
        tm = _hip.Timing()
        if _lib.ptowsp_hip_synchronize(self.prog._h, ctypes.byref(tm)) != 0:
            raise RuntimeError(_hip._error())
        res = _hip.RunInfo()
        assert _lib.ptowsp_hip_run_result(self.prog._h, ctypes.byref(res)) == 0
        return int(res.total_cycles), int(res.task_count)


def _reset(t):
    t["m"].fill_(float("-inf"))
    t["l"].zero_()
    t["o"].zero_()
    t["out"].zero_()


def _decode_case(gpu, batch, lmax, seed):
    t = W.paged_decode_torch(gpu, batch=batch, hq=32, hkv=8, d=128, lmin=1, lmax=lmax, seed=seed)
    return t, AbiProgram(W.rr4(W.paged_decode(t)), f"noalloc_decode_{batch}")


def test_noalloc_decode_matches_launch_twice(gpu):
    import torch

    # First call: the full-size batch; second call: a smaller input (fewer sequences, shorter).
    for batch, lmax, seed in ((64, 4096, 11), (8, 700, 12)):
        t, p = _decode_case(gpu, batch, lmax, seed)
        print(f"no-alloc decode: batch {batch}, lengths <= {lmax}", flush=True)
        _reset(t)
        ref_cycles = p.run(_lib.ptowsp_hip_launch)
        ref = t["out"].clone()
        assert torch.isfinite(ref).all()
        # Leave garbage in the outputs and accumulators' neighbours: the run must not depend on them.
        _reset(t)
        t["out"].fill_(123.0)
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info(gpu)[0]
        got_cycles = p.run(_lib.ptowsp_hip_launch_noalloc)
        torch.cuda.synchronize()
        free_after = torch.cuda.mem_get_info(gpu)[0]
        assert free_after == free_before, (free_before, free_after)
        assert torch.equal(t["out"], ref)
        assert got_cycles == ref_cycles
        # The existing entry point is unaffected by the no-allocation run in between.
        _reset(t)
        assert p.run(_lib.ptowsp_hip_launch) == ref_cycles
        assert torch.equal(t["out"], ref)
        # The decode against float64 attention (the north-star bound for bf16 attention).
        h = {k: (v.view(torch.int16).cpu().numpy().view(np.uint16) if v.dtype == torch.bfloat16 else v.cpu().numpy())
             for k, v in t.items() if k != "lengths"}
        h["lengths"] = t["lengths"]
        want = W.paged_decode_ref(h)
        rel = np.linalg.norm(t["out"].cpu().numpy() - want) / np.linalg.norm(want)
        assert rel <= 1e-2, rel


def test_noalloc_refuses_oversized_scratch(gpu):
    """A decode launch whose counters + partials exceed the fixed 16 MiB scratch is refused."""
    import torch

    t = W.paged_decode_torch(gpu, batch=512, hq=64, hkv=8, d=128, lmin=16, lmax=32, seed=3)
    p = AbiProgram(W.rr4(W.paged_decode(t)), "noalloc_big")
    _reset(t)
    p.run(_lib.ptowsp_hip_launch)  # builds and loads the kernels; allocates its own scratch
    ref = t["out"].clone()
    _reset(t)
    with pytest.raises(RuntimeError, match="bytes of scratch"):
        p.run(_lib.ptowsp_hip_launch_noalloc)
    torch.cuda.synchronize()
    # The program is still usable through the allocating entry point.
    _reset(t)
    p.run(_lib.ptowsp_hip_launch)
    assert torch.equal(t["out"], ref)


def test_noalloc_refuses_host_tensors(gpu):
    x = np.random.default_rng(0).standard_normal((1, 2, 16, 128), dtype=np.float32)
    p = AbiProgram(W.rr4(W.rmsnorm({"x": x, "y": np.zeros_like(x)})), "noalloc_host")
    with pytest.raises(RuntimeError, match="host memory"):
        p.run(_lib.ptowsp_hip_launch_noalloc)
