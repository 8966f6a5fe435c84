"""BASELINE.json configurations at full size on the GPU, checked against the
oracle over every element, plus size-independent invariants of the math.

rmsnorm_tile over X[16,8192,16,128] f32 ~ N(0,1)  (1 GiB in)
row softmax over X[8,4096,32,512] f32 ~ N(0,3)    (2 GiB in)
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu


def _close(got, ref, rtol, atol):
    """Elementwise |got-ref| <= atol + rtol*|ref| on the GPU; returns the worst ratio."""
    import torch

    err = (got - ref).abs()
    tol = atol + rtol * ref.abs()
    worst = float((err / tol.clamp_min(1e-38)).max())
    return bool((err <= tol).all()), worst


def _run(kind, shape, sigma, seed):
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * sigma
    y = torch.empty_like(x)
    make = W.rmsnorm if kind == "rmsnorm" else W.softmax
    prog = W.rr4(make({"x": x, "y": y})).compile(target="hip_gfx950")
    prog.execute()
    prog.synchronize()
    xh = x.cpu().numpy()
    yh = np.zeros_like(xh)
    ref = run_workload(W.rr4(make({"x": xh, "y": yh})))
    return x, y, torch.from_numpy(yh).to(dev), prog, ref


def test_config1_rmsnorm_bandwidth_full(gpu):
    import torch

    x, y, yref, prog, ref = _run("rmsnorm", (16, 8192, 16, 128), 1.0, 0)
    ok, worst = _close(y, yref, 1e-5, 1e-6)
    assert ok, f"worst |err|/tol = {worst}"
    assert prog.stats.task_count == ref.task_count == 16 * 8192
    assert prog.stats.total_cycles == ref.total_cycles == 270_008_320
    # Invariant: every output row has mean square 1.
    ms = (y.double() ** 2).mean(dim=-1)
    assert float((ms - 1.0).abs().max()) < 1e-5
    del x, y, yref
    torch.cuda.empty_cache()


def test_config2_softmax_full(gpu):
    import torch

    x, y, yref, prog, ref = _run("softmax", (8, 4096, 32, 512), 3.0, 0)
    ok, worst = _close(y, yref, 1e-5, 0.0)
    assert ok, f"worst |err|/tol = {worst}"
    assert prog.stats.total_cycles == ref.total_cycles
    # Invariants: rows sum to 1; the row maximum maps to 1/rowsum.
    s = y.double().sum(dim=-1)
    assert float((s - 1.0).abs().max()) < 1e-5
    assert float(y.min()) >= 0.0
    del x, y, yref
    torch.cuda.empty_cache()
