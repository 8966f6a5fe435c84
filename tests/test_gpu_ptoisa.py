"""GPU parity for @ptoisa_kernel and the top-k ops (the reference's tests/test_ptoisa_kernel_jit.py:22-95).

Each case runs on the HIP target and on the CPU oracle (pinned against numpy
in tests/test_ptoisa.py) and requires identical results and cycle totals:
bit-exact for the sort indices and for every op that is one correctly rounded
fp32 operation; exp / rsqrt within 2 ulp.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from test_ptoisa import mix_arrays, mix_expected, tie_scores

pytestmark = pytest.mark.gpu


def _hip(w):
    prog = w.compile(target="hip_gfx950")
    prog.execute()
    prog.synchronize()
    return prog


def _pair(make, arrs, window):
    ga = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in arrs.items()}
    ca = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in arrs.items()}
    prog = _hip(W.rr2(make(ga), window))
    ref = run_workload(W.rr2(make(ca), window))
    assert prog.stats.total_cycles == ref.total_cycles
    return ga, ca, prog


def test_ptoisa_square_tile(gpu):
    """tests/test_ptoisa_kernel_jit.py:22-54."""
    x = np.random.default_rng(0).standard_normal((4, 1, 32, 32), dtype=np.float32)
    ga, ca, prog = _pair(W.ptoisa_square, {"x": x, "y": np.zeros_like(x)}, 2048)
    np.testing.assert_array_equal(ga["y"], x * x)
    np.testing.assert_array_equal(ga["y"], ca["y"])
    assert prog.stats.total_cycles == 6144


def test_ptoisa_tsort32_topk_indices(gpu):
    """tests/test_ptoisa_kernel_jit.py:57-95."""
    scores = np.random.default_rng(0).standard_normal((2, 3, 1, 32), dtype=np.float32)
    arrs = {"scores": scores, "out": np.zeros((2, 3, 1, 8), np.int32)}
    ga, ca, prog = _pair(W.ptoisa_topk, arrs, 4096)
    want = np.argsort(-scores.reshape(2, 3, 32), axis=-1)[:, :, :8].astype(np.int32)
    np.testing.assert_array_equal(ga["out"].reshape(2, 3, 8), want)
    np.testing.assert_array_equal(ga["out"], ca["out"])
    assert prog.stats.total_cycles == 576


def test_tsort32_ties_signed_zero_and_nan(gpu):
    s = tie_scores(64, 9)
    arrs = {"scores": s, "out": np.zeros((64, 1, 1, 32), np.int32)}
    ga, ca, _ = _pair(lambda a: W.ptoisa_topk(a, k=32), arrs, 4096)
    want = np.argsort(-s.reshape(64, 32), axis=-1, kind="stable").astype(np.int32)
    np.testing.assert_array_equal(ga["out"].reshape(64, 32), want)
    np.testing.assert_array_equal(ga["out"], ca["out"])


def test_topk_store_leaves_other_columns(gpu):
    scores = np.random.default_rng(3).standard_normal((1, 2, 1, 32), dtype=np.float32)
    arrs = {"scores": scores, "out": np.full((1, 2, 1, 12), -7, np.int32)}
    ga, ca, _ = _pair(lambda a: W.ptoisa_topk(a, k=5), arrs, 64)
    np.testing.assert_array_equal(ga["out"], ca["out"])
    assert (ga["out"].reshape(2, 12)[:, 5:] == -7).all()


def test_pto_tracer_topk(gpu):
    scores = np.random.default_rng(4).standard_normal((4, 50, 1, 32), dtype=np.float32)
    arrs = {"scores": scores, "out": np.zeros((4, 50, 1, 8), np.int32)}
    ga, ca, _ = _pair(W.pto_topk, arrs, 4096)
    want = np.argsort(-scores.reshape(4, 50, 32), axis=-1)[:, :, :8]
    np.testing.assert_array_equal(ga["out"].reshape(4, 50, 8), want)
    np.testing.assert_array_equal(ga["out"], ca["out"])


def test_ptoisa_instruction_mix(gpu):
    a = mix_arrays(B=5)
    ga, ca, _ = _pair(lambda d: W.ptoisa_mix(d, extra_cycles=7), a, 64)
    np.testing.assert_array_equal(ga["out"], mix_expected(a))
    np.testing.assert_array_equal(ga["out"], ca["out"])


def test_ptoisa_exp_rsqrt(gpu):
    x = np.random.default_rng(5).uniform(-4, 4, (3, 8, 64)).astype(np.float32)
    ga, ca, _ = _pair(W.ptoisa_unary, {"x": x, "out": np.zeros_like(x)}, 64)
    np.testing.assert_allclose(ga["out"], ca["out"], rtol=2.4e-7, atol=0)


@pytest.mark.parametrize("impl,cycles", [("pto", 800), ("ptoisa", 1319680)])
def test_lightning_indexer_example(gpu, impl, cycles):
    """examples/deepseek_lightning_indexer (its seed-0 inputs): golden top-8 indices and the
    cycles the example records for its pto / ptoisa kernels."""
    scores, eff = W.lightning_inputs()
    out = np.zeros((2, 4, 1, 8), np.int32)
    prog = _hip(W.lightning_indexer(scores, eff, out, impl))
    np.testing.assert_array_equal(out.reshape(2, 4, 8), W.stable_topk_desc(scores, 8))
    assert prog.stats.total_cycles == cycles


@pytest.mark.parametrize("impl", ["pto", "ptoisa"])
def test_lightning_indexer_larger(gpu, impl):
    scores, eff = W.lightning_inputs(seed=3, bsz=8, tiles=64)
    out = np.zeros((8, 64, 1, 8), np.int32)
    prog = _hip(W.lightning_indexer(scores, eff, out, impl))
    ref_out = np.zeros_like(out)
    ref = run_workload(W.lightning_indexer(scores, eff, ref_out, impl))
    np.testing.assert_array_equal(out.reshape(8, 64, 8), W.stable_topk_desc(scores, 8))
    np.testing.assert_array_equal(out, ref_out)
    assert prog.stats.total_cycles == ref.total_cycles
